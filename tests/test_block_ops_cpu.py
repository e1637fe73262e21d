"""Contract checks of the page-level KV movement functions, without a GPU.

Error types and messages follow the reference runner
(prism_infer/engine/model_runner.py:917-1031): prefix rows outside
[1, block_size] raise ValueError, a bad swap direction ValueError, a missing
CPU cache or unpaired scale caches RuntimeError.  Valid CPU tensors reach the
device path and raise (there is no CPU fallback).
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


def test_copies_have_no_cpu_fallback():
    kv, sc = _caches()
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        copy_kv_blocks(kv, [(0, 1)], sc)
