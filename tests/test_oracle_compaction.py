"""Pins the oracle's slot compaction (oracle/kv_oracle.c) on the CPU.

Reference: ``compact_kv_slots`` (prism_infer/ops/kv_compaction.py:93-112):
every destination slot receives what its source slot held before the call.
Checked against torch's ``index_select`` / ``index_copy_`` (the reference's own
non-FP8 formulation, :111-112), against the reference test's plan
(tests/test_kv_physical_layout.py:411-453 and :703-759: P = 4, tokens
[0, 1, 2, 7, 8, 9] kept in place) and against the read-before-write invariant
when sources and destinations overlap (forward and backward shifts, swaps,
cycles), where a naive in-order copy gives a different answer.
"""

from __future__ import annotations

import pytest
import torch

from oracle import compact_slots, compact_slots_torch
from prism_infer.engine.kv_compaction_plan import plan_in_place

FP8 = torch.float8_e4m3fn


def _cache(seed, rows_kv=2, layers=2, slots=32, tail=(1, 8), dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows_kv, layers, slots, *tail, generator=g)
    return x.to(dtype)


def _bytes(t):
    return t.contiguous().view(torch.uint8) if t.element_size() == 1 else t.contiguous().view(-1).view(torch.uint8)


def _naive_in_order(cache, src, dst):
    out = cache.clone()
    for s, d in zip(src.tolist(), dst.tolist()):
        out[:, :, d] = out[:, :, s]
    return out


def test_reference_plan_in_place_known_answer():
    plan = plan_in_place([0, 1, 2], [0, 1, 2, 7, 8, 9], 4, logical_prompt_len=10)
    assert plan.source_slots == (0, 1, 2, 7, 8, 9)
    assert plan.destination_slots == (0, 1, 2, 3, 4, 5)
    assert plan.new_block_table == (0, 1) and plan.released_block_ids == (2,)
    assert plan.physical_prompt_len == 6
    torch.manual_seed(20260711)
    cache = torch.randn(2, 2, 8, 4, 1, 8, dtype=torch.bfloat16).to(FP8)
    flat = cache.view(2, 2, -1, 1, 8)
    src, dst = plan.tensors("cpu")
    expected = flat.view(torch.uint8).index_select(2, src).clone()
    compact_slots(flat, src, dst)
    assert torch.equal(flat.view(torch.uint8).index_select(2, dst), expected)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, FP8])
@pytest.mark.parametrize("pattern", ["disjoint", "shift_down", "shift_up", "swap", "cycle", "identity"])
def test_matches_index_select_copy(dtype, pattern):
    slots = 32
    cache = _cache(7, slots=slots, dtype=dtype if dtype != FP8 else torch.bfloat16)
    if dtype == FP8:
        cache = cache.to(FP8)
    g = torch.Generator().manual_seed(1)
    if pattern == "disjoint":
        src = torch.arange(0, 10)
        dst = torch.arange(20, 30)
    elif pattern == "shift_down":
        src = torch.arange(3, 19)
        dst = torch.arange(0, 16)
    elif pattern == "shift_up":
        src = torch.arange(0, 16)
        dst = torch.arange(5, 21)
    elif pattern == "swap":
        src = torch.tensor([4, 9])
        dst = torch.tensor([9, 4])
    elif pattern == "cycle":
        src = torch.randperm(slots, generator=g)
        dst = torch.roll(src, 1)
    else:
        src = dst = torch.randperm(slots, generator=g)[:12]
    want = cache.view(torch.uint8).clone() if dtype == FP8 else cache.clone()
    compact_slots_torch(want, src, dst)
    got = cache.clone()
    compact_slots(got, src, dst)
    assert torch.equal(_bytes(got), _bytes(want))
    if pattern in ("shift_up", "swap", "cycle"):
        # a naive in-order copy reads already-overwritten sources here
        assert not torch.equal(_bytes(_naive_in_order(cache, src, dst)), _bytes(want))


def test_scale_cache_and_payload_move_together():
    """Payload [2, L, S, H, D] and scales [2, L, S, H] moved by the same slot lists (test_scaled_fp8_kv_cache.py:322-344)."""

    g = torch.Generator().manual_seed(4)
    payload = torch.randn(2, 3, 40, 2, 8, generator=g).to(FP8)
    scales = torch.rand(2, 3, 40, 2, generator=g)
    plan = plan_in_place(list(range(10)), sorted(torch.randperm(40, generator=g)[:17].tolist()), 4,
                         logical_prompt_len=40)
    src, dst = plan.tensors("cpu")
    p_want = payload.view(torch.uint8).index_select(2, src).clone()
    s_want = scales.index_select(2, src).clone()
    compact_slots(payload, src, dst)
    compact_slots(scales, src, dst)
    assert torch.equal(payload.view(torch.uint8).index_select(2, dst), p_want)
    assert torch.equal(scales.index_select(2, dst), s_want)


def test_untouched_slots_and_out_of_range():
    cache = _cache(9, slots=16)
    before = cache.clone()
    src = torch.tensor([1, 2, 3])
    dst = torch.tensor([10, 11, 12])
    compact_slots(cache, src, dst)
    others = [i for i in range(16) if i not in (10, 11, 12)]
    assert torch.equal(cache[:, :, others], before[:, :, others])
    with pytest.raises(IndexError):
        compact_slots(cache, torch.tensor([0, 16]), torch.tensor([1, 2]))
