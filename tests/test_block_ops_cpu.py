"""Contract checks of the page-level KV movement functions, without a GPU.

Error types and messages follow the reference runner
(prism_infer/engine/model_runner.py:917-1031): prefix rows outside
[1, block_size] raise ValueError, a bad swap direction ValueError, a missing
CPU cache or unpaired scale caches RuntimeError.  Valid CPU caches go through
``compact_kv_slots``'s CPU branch, like the reference's torch copies.
"""

from __future__ import annotations

import pytest
import torch

from prism_infer.engine.kv_block_ops import copy_kv_block_prefixes, copy_kv_blocks, swap_blocks


def _caches():
    return torch.zeros(2, 1, 4, 4, 1, 2), torch.zeros(2, 1, 4, 4, 1)


def test_prefix_rows_range():
    kv, sc = _caches()
    with pytest.raises(ValueError, match=r"rows must be in \[1, 4\]"):
        copy_kv_block_prefixes(kv, [(0, 1, 0)], sc)
    with pytest.raises(ValueError, match=r"rows must be in \[1, 4\]"):
        copy_kv_block_prefixes(kv, [(0, 1, 5)], sc)


def test_block_ids_and_shapes():
    kv, sc = _caches()
    with pytest.raises(ValueError, match="block ids"):
        copy_kv_blocks(kv, [(0, 4)], sc)
    with pytest.raises(ValueError, match="without head_dim"):
        copy_kv_blocks(kv, [(0, 1)], sc[..., :1, :])
    with pytest.raises(ValueError, match=r"\[2, layers, blocks"):
        copy_kv_blocks(kv[0], [(0, 1)])


def test_empty_inputs_are_no_ops():
    kv, sc = _caches()
    copy_kv_blocks(kv, [], sc)
    copy_kv_block_prefixes(kv, [], sc)
    swap_blocks(kv, None, [], "sideways")


def test_swap_contract():
    kv, sc = _caches()
    with pytest.raises(ValueError, match="direction"):
        swap_blocks(kv, kv.clone(), [(0, 0)], "sideways")
    with pytest.raises(RuntimeError, match="without an allocated CPU payload cache"):
        swap_blocks(kv, None, [(0, 0)], "out")
    with pytest.raises(RuntimeError, match="both exist or both be absent"):
        swap_blocks(kv, kv.clone(), [(0, 0)], "out", gpu_scale_cache=sc)
    with pytest.raises(RuntimeError, match="between a GPU cache and a CPU cache"):
        swap_blocks(kv, kv.clone(), [(0, 0)], "out")


def test_copies_on_cpu_caches():
    kv, sc = _caches()
    kv[:, :, 0].copy_(torch.randn(2, 1, 4, 1, 2))
    sc[:, :, 0].copy_(torch.randn(2, 1, 4, 1))
    copy_kv_blocks(kv, [(0, 1)], sc)
    assert torch.equal(kv[:, :, 1], kv[:, :, 0]) and torch.equal(sc[:, :, 1], sc[:, :, 0])
    copy_kv_block_prefixes(kv, [(0, 2, 3)], sc)
    assert torch.equal(kv[:, :, 2, :3], kv[:, :, 0, :3]) and bool((kv[:, :, 2, 3] == 0).all())
    assert torch.equal(sc[:, :, 2, :3], sc[:, :, 0, :3])
