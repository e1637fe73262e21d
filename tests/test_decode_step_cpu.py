"""Host logic of the decode step: the packed metadata layout of the
reference's input preparation (prism_infer/engine/input_preparation.py:571-603)
and the cache-binding checks of its Attention layer (layers/attention.py:115-140)."""

from __future__ import annotations

import pytest
import torch

from prism_infer.engine.decode_attention import PagedKVDecodeAttention, pack_decode_metadata


def test_packed_layout_and_views_share_storage():
    m = pack_decode_metadata([5, -1, 9], [6, 0, 10], [[1], [], [2, 3]], logical_context_lens=[7, 0, 12])
    assert m.packed.tolist() == [5, -1, 9, 6, 0, 10, 7, 0, 12, 10, 1, -1, -1, -1, 2, 3]
    assert m.block_tables.tolist() == [[1, -1], [-1, -1], [2, 3]]
    assert m.max_context_len.ndim == 0 and int(m.max_context_len) == 10
    ptr = m.packed.data_ptr()
    assert m.slot_mapping.data_ptr() == ptr
    assert m.context_lens.data_ptr() == ptr + 3 * 4
    assert m.block_tables.data_ptr() == ptr + 10 * 4
    other = pack_decode_metadata([1, 2, 3], [4, 5, 6], [[7], [8], [9, 9]])
    m.copy_(other)
    assert m.slot_mapping.tolist() == [1, 2, 3] and m.block_tables.tolist() == [[7, -1], [8, -1], [9, 9]]
    with pytest.raises(ValueError, match="layouts differ"):
        m.copy_(pack_decode_metadata([1], [2], [[3]]))
    with pytest.raises(ValueError, match="longer than the width"):
        pack_decode_metadata([1], [2], [[3, 4, 5]], width=2)


def test_binding_checks_match_reference_messages():
    layer = PagedKVDecodeAttention(4, 2, 8, 0.3)
    meta = pack_decode_metadata([0], [1], [[0]])
    q, k = torch.zeros(1, 4, 8), torch.zeros(1, 2, 8)
    with pytest.raises(RuntimeError, match="requires bound K/V caches"):
        layer(q, k, k, meta)
    layer.k_cache = torch.zeros(1, 4, 2, 8, dtype=torch.float8_e4m3fn)
    with pytest.raises(RuntimeError, match="payload caches must be bound together"):
        layer(q, k, k, meta)
    layer.v_cache = torch.zeros_like(layer.k_cache)
    layer.k_scale_cache = torch.zeros(1, 4, 2)
    with pytest.raises(RuntimeError, match="scale caches must be bound together"):
        layer(q, k, k, meta)
    layer.v_scale_cache = torch.zeros(1, 4, 2)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        layer(q, k, k, meta)
    with pytest.raises(ValueError, match="divisible"):
        PagedKVDecodeAttention(5, 2, 8, 0.3)
