"""One attention layer's decode step on the scaled-FP8 paged KV cache.

Restates the decode branch of the reference's ``Attention`` layer
(prism_infer/layers/attention.py:85-111 routing, :115-156 cache-binding
checks, :158-169 ``_store_current_kv``, :350-371
``_forward_decode_paged_triton``): store the step's K/V into their slots,
then paged decode attention over the pages, with ``max_context_len`` from
the step's metadata.

Decode metadata is packed the way the reference's input preparation packs
it (prism_infer/engine/input_preparation.py:571-603): one int32 buffer
``[B slot][B ctx][B logical ctx][1 max ctx][B * W block table]`` whose
slices are the kernels' inputs.  A graph captured over a layer keeps reading
that buffer, so refilling it in place (:meth:`DecodeMetadata.copy_`) is all a
replay needs; padded rows use ``slot = -1`` and ``ctx = 0`` (skipped by the
store, zero output from the decode).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from prism_infer.ops.kv_cache_store import store_kvcache
from prism_infer.ops.paged_decode import paged_decode_attention


@dataclass
class DecodeMetadata:
    packed: torch.Tensor          # int32 [3 * B + 1 + B * W]
    slot_mapping: torch.Tensor    # int32 [B]
    context_lens: torch.Tensor    # int32 [B] (physical KV length)
    logical_context_lens: torch.Tensor
    max_context_len: torch.Tensor  # int32, 0-dim
    block_tables: torch.Tensor    # int32 [B, W]

    @property
    def batch(self) -> int:
        return self.slot_mapping.numel()

    def copy_(self, other: "DecodeMetadata") -> "DecodeMetadata":
        """Refill this buffer from ``other`` (same batch and width), in place."""

        if other.packed.shape != self.packed.shape or other.block_tables.shape != self.block_tables.shape:
            raise ValueError("decode metadata layouts differ")
        self.packed.copy_(other.packed, non_blocking=True)
        return self


def pack_decode_metadata(slot_mapping, context_lens, block_tables, *, logical_context_lens=None,
                         width: int | None = None, device=None) -> DecodeMetadata:
    """Pack one decode step's metadata into a single int32 buffer on ``device``.

    ``block_tables`` is a list of per-sequence block id lists (padded with -1
    to ``width``, default the longest) or an int tensor ``[B, W]``.
    """

    slots = [int(s) for s in slot_mapping]
    lens = [int(c) for c in context_lens]
    logical = lens if logical_context_lens is None else [int(c) for c in logical_context_lens]
    batch = len(slots)
    if len(lens) != batch or len(logical) != batch:
        raise ValueError("slot_mapping, context_lens and logical_context_lens must have one entry per sequence")
    if isinstance(block_tables, torch.Tensor):
        rows = [[int(x) for x in row] for row in block_tables.tolist()]
    else:
        rows = [[int(x) for x in row] for row in block_tables]
    if len(rows) != batch:
        raise ValueError("block_tables must have one row per sequence")
    w = max((len(r) for r in rows), default=0) if width is None else int(width)
    if any(len(r) > w for r in rows):
        raise ValueError(f"a block table is longer than the width {w}")
    flat = [x for r in rows for x in (r + [-1] * (w - len(r)))]
    values = [*slots, *lens, *logical, max(lens, default=0), *flat]
    packed = torch.tensor(values, dtype=torch.int32, device=device)
    o = 0
    slot_t = packed[o:o + batch]
    o += batch
    ctx_t = packed[o:o + batch]
    o += batch
    logical_t = packed[o:o + batch]
    o += batch
    max_t = packed[o]
    o += 1
    tables_t = packed[o:].view(batch, w)
    return DecodeMetadata(packed, slot_t, ctx_t, logical_t, max_t, tables_t)


class PagedKVDecodeAttention:
    """Decode attention of one layer over its (scaled-)FP8 paged KV cache.

    Bind the layer's caches to ``k_cache`` / ``v_cache`` ([blocks, page,
    kv_heads, head_dim]) and, for the scaled format, ``k_scale_cache`` /
    ``v_scale_cache`` ([blocks, page, kv_heads] fp32), as the reference's
    model runner does (model_runner.py:817-837).
    """

    def __init__(self, num_heads: int, num_kv_heads: int, head_dim: int, scale: float):
        if num_heads % num_kv_heads:
            raise ValueError(f"num_heads must be divisible by num_kv_heads, got {num_heads} and {num_kv_heads}")
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.scale = scale
        self.k_cache = torch.tensor([])
        self.v_cache = torch.tensor([])
        self.k_scale_cache: torch.Tensor | None = None
        self.v_scale_cache: torch.Tensor | None = None

    def _validate_cache_bindings(self) -> None:
        """The reference's binding checks (attention.py:115-140)."""

        if (self.k_scale_cache is None) != (self.v_scale_cache is None):
            raise RuntimeError("attention K/V scale caches must be bound together")
        k_bound, v_bound = bool(self.k_cache.numel()), bool(self.v_cache.numel())
        if k_bound != v_bound:
            raise RuntimeError("attention K/V payload caches must be bound together")
        if not k_bound:
            raise RuntimeError("paged decode requires bound K/V caches")
        if self.k_scale_cache is not None and (not self.k_scale_cache.numel() or not self.v_scale_cache.numel()):
            raise RuntimeError("bound K/V scale caches must not be empty")

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, metadata: DecodeMetadata) -> torch.Tensor:
        """Store the step's K/V ([B, kv_heads, head_dim]) and attend; q is [B, num_heads, head_dim]."""

        self._validate_cache_bindings()
        if metadata.slot_mapping is None:
            raise RuntimeError("bound KV cache requires slot_mapping")
        store_kvcache(k, v, self.k_cache, self.v_cache, metadata.slot_mapping, self.k_scale_cache,
                      self.v_scale_cache)
        return paged_decode_attention(
            q, self.k_cache, self.v_cache, metadata.block_tables, metadata.context_lens, self.scale,
            k_scale_cache=self.k_scale_cache, v_scale_cache=self.v_scale_cache,
            max_context_len=metadata.max_context_len,
        )

    __call__ = forward


__all__ = ["DecodeMetadata", "PagedKVDecodeAttention", "pack_decode_metadata"]
