"""Host-side logic of the KV path on the CPU: format constants, byte accounting,
compaction slot plans, synthetic workloads and the bench contract guard.

Known answers come from the reference: storage ratios 0.5 / 0.015625 /
0.515625 (tests/test_scaled_fp8_kv_cache.py:124-146), the compaction plan of
tests/test_kv_physical_layout.py:411-453, and the algorithmic byte formulas of
the measured configurations (2112 B per token-layer; 4,341,796 B for one
2048-token sequence; 50,888,704 B for the 8192-token store).
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest
import torch

from prism_infer import workloads
from prism_infer.engine.kv_compaction_plan import plan_in_place, plan_out_of_place
from prism_infer.engine.kv_quantization import (
    FP8_E4M3FN_MAX,
    KV_SCALE_DTYPE,
    PER_TOKEN_HEAD_SCALE_FLOOR,
    KVStorageBytes,
    kv_block_storage_bytes,
    kv_cache_storage_bytes,
    kv_token_layer_bytes,
    scale_cache_shape,
    tensor_storage_bytes,
)

REPO = Path(__file__).resolve().parents[1]


def test_format_constants():
    assert FP8_E4M3FN_MAX == 448.0
    assert PER_TOKEN_HEAD_SCALE_FLOOR == 1.0e-6
    assert KV_SCALE_DTYPE is torch.float32
    assert float(torch.finfo(torch.float8_e4m3fn).max) == FP8_E4M3FN_MAX


def test_storage_ratios_match_reference():
    shape = dict(num_layers=36, page_size=256, num_kv_heads=8, head_dim=128)
    bf16 = kv_block_storage_bytes(**shape, payload_dtype=torch.bfloat16, token_head_scales=False)
    fp8 = kv_block_storage_bytes(**shape, payload_dtype=torch.float8_e4m3fn, token_head_scales=True)
    assert fp8.payload / bf16.total == 0.5
    assert fp8.scales / bf16.total == 0.015625
    assert fp8.total / bf16.total == 0.515625
    assert fp8.total == 19_464_192
    assert kv_token_layer_bytes(num_kv_heads=8, head_dim=128) == 2112
    assert kv_token_layer_bytes(num_kv_heads=8, head_dim=128, token_head_scales=False) == 2048


def test_scale_cache_shape_and_errors():
    assert scale_cache_shape((10, 256, 8, 128)) == (10, 256, 8)
    assert scale_cache_shape((100, 8, 128)) == (100, 8)
    with pytest.raises(ValueError):
        scale_cache_shape((8, 128))
    with pytest.raises(ValueError):
        scale_cache_shape((0, 256, 8, 128))
    with pytest.raises(ValueError):
        kv_block_storage_bytes(num_layers=0, page_size=256, num_kv_heads=8, head_dim=128,
                               payload_dtype=torch.bfloat16, token_head_scales=False)


def test_allocated_cache_bytes_equal_pages_times_block_bytes():
    # The engine's cache is [K|V, layers, blocks, page, heads, dim] with scales
    # [K|V, layers, blocks, page, heads] (model_runner.py:817-837); its bytes must be
    # num_blocks times the per-block figure, and one block's slice (the view
    # bench_system.py:574 measures) exactly the per-block figure.
    L, N, P, H, D = 3, 5, 16, 4, 32
    payload = torch.empty((2, L, N, P, H, D), dtype=torch.float8_e4m3fn)
    scales = torch.empty((2, L, N, P, H), dtype=torch.float32)
    per_block = kv_block_storage_bytes(num_layers=L, page_size=P, num_kv_heads=H, head_dim=D,
                                       payload_dtype=torch.float8_e4m3fn, token_head_scales=True)
    whole = kv_cache_storage_bytes(payload, scales)
    assert isinstance(whole, KVStorageBytes)
    assert whole == KVStorageBytes(N * per_block.payload, N * per_block.scales)
    assert tensor_storage_bytes(payload[:, :, 0]) == per_block.payload
    assert tensor_storage_bytes(scales[:, :, 0]) == per_block.scales
    dense = torch.empty((2, L, N, P, H, D), dtype=torch.bfloat16)
    assert kv_cache_storage_bytes(dense, None) == KVStorageBytes(dense.numel() * 2, 0)
    assert tensor_storage_bytes(None) == 0
    with pytest.raises(TypeError):
        tensor_storage_bytes([1, 2])
    with pytest.raises(TypeError):
        kv_cache_storage_bytes(None, scales)
    with pytest.raises(TypeError):
        kv_block_storage_bytes(num_layers=1, page_size=1, num_kv_heads=1, head_dim=1,
                               payload_dtype="fp8", token_head_scales=True)
    with pytest.raises(ValueError):
        kv_block_storage_bytes(num_layers=True, page_size=1, num_kv_heads=1, head_dim=1,
                               payload_dtype=torch.bfloat16, token_head_scales=False)


def test_in_place_plan_reference_case():
    plan = plan_in_place([0, 1, 2], [0, 1, 2, 7, 8, 9], 4, logical_prompt_len=10)
    assert plan.source_slots == (0, 1, 2, 7, 8, 9)
    assert plan.destination_slots == (0, 1, 2, 3, 4, 5)
    assert plan.new_block_table == (0, 1)
    assert plan.released_block_ids == (2,)
    assert (plan.physical_prompt_len, plan.final_physical_prompt_len) == (6, 6)


def test_in_place_plan_scattered_pages_and_text_tail():
    # pages [5, 2, 9], keep 0, 3, 6 of a 7-token compacted prefix; 2 uncompacted text tokens follow
    plan = plan_in_place([5, 2, 9], [0, 3, 6], 4, logical_prompt_len=9, compacted_logical_len=7)
    assert plan.source_slots == (20, 23, 10)
    assert plan.destination_slots == (20, 21, 22)
    assert plan.final_physical_prompt_len == 5
    assert plan.new_block_table == (5, 2) and plan.released_block_ids == (9,)


def test_plan_validation():
    with pytest.raises(RuntimeError):
        plan_in_place([0, 1], [], 4, logical_prompt_len=8)
    with pytest.raises(ValueError):
        plan_in_place([0, 1], [3, 1], 4, logical_prompt_len=8)
    with pytest.raises(ValueError):
        plan_in_place([0, 1], [1, 8], 4, logical_prompt_len=8)
    with pytest.raises(RuntimeError):
        plan_in_place([0], [0, 1], 4, logical_prompt_len=8)
    with pytest.raises(ValueError):
        plan_out_of_place([0, 1], [0, 5], 4, [1])


def test_in_place_plan_refuses_shared_pages():
    # kv_compaction_coordinator.py:49-58: pages with ref_count != 1 are never rewritten
    counts = {4: 1, 6: 2, 8: 1}
    with pytest.raises(RuntimeError, match=r"prefix-shared blocks; shared_block_ids=\[6\]"):
        plan_in_place([4, 6, 8], [0, 5], 4, logical_prompt_len=12, ref_counts=counts)
    with pytest.raises(RuntimeError, match="shared_block_ids=\\[4, 8\\]"):
        plan_in_place([4, 6, 8], [0, 5], 4, logical_prompt_len=12,
                      ref_counts=lambda b: 1 if b == 6 else 0)
    plan = plan_in_place([4, 6, 8], [0, 5], 4, logical_prompt_len=12, ref_counts={4: 1, 6: 1, 8: 1})
    assert plan.source_slots == (16, 25) and plan.destination_slots == (16, 17)
    # the out-of-place plan only reads the old pages, so sharing them is allowed
    assert plan_out_of_place([4, 6], [1], 4, [9]).destination_slots == (36,)


def test_plan_validate_catches_tampering():
    import dataclasses

    plan = plan_in_place([5, 2, 9], [0, 3, 6], 4, logical_prompt_len=9, compacted_logical_len=7)
    plan.validate(4)
    bad = {
        "plan must compact into the existing page-table prefix": dict(new_block_table=(2, 5)),
        "plan released blocks must be the old page-table suffix": dict(released_block_ids=()),
        "plan compact block count is inconsistent": dict(new_block_table=(5,)),
        "plan destination slots are not a dense physical tail": dict(destination_slots=(20, 21, 23)),
        "physical prompt length must equal source slots": dict(source_slots=(20, 23)),
        "plan retained positions must be sorted and unique": dict(retained_positions=(0, 6, 3)),
        "plan retained positions exceed compacted prefix": dict(retained_positions=(0, 3, 7)),
        "compacted logical prefix is outside prompt bounds": dict(compacted_logical_len=10),
        "plan source slots do not follow the retained positions": dict(source_slots=(20, 23, 11)),
    }
    for message, change in bad.items():
        with pytest.raises(ValueError, match=message):
            dataclasses.replace(plan, **change).validate(4)
    with pytest.raises(ValueError, match="negative block id"):
        plan_in_place([0, -1], [0], 4, logical_prompt_len=8)
    with pytest.raises(ValueError, match="names a block twice"):
        plan_in_place([3, 3], [0], 4, logical_prompt_len=8)
    with pytest.raises(ValueError, match="names a block twice"):
        plan_out_of_place([0, 1], [0, 1, 2, 3, 4], 4, [7, 7])


def test_out_of_place_plan_is_disjoint():
    plan = plan_out_of_place([3, 7], [1, 2, 4, 6], 4, [10, 11])
    assert plan.source_slots == (13, 14, 28, 30)
    assert plan.destination_slots == (40, 41, 42, 43)
    assert not set(plan.source_slots) & set(plan.destination_slots)


def test_mixed_workload_metadata_and_bytes():
    w = workloads.decode_mixed("cpu", fill=False)
    lens = w.context_lens.tolist()
    tables = w.block_tables
    assert len(lens) == 64 and all(1024 <= n <= 16384 for n in lens)
    sharing = w.meta["sharing"]
    assert len(sharing) == 32
    # the 32 longest share the same 16 leading pages; nobody else uses them
    longest = sorted(range(64), key=lambda b: -lens[b])[:32]
    assert sorted(longest) == sharing or min(lens[b] for b in sharing) >= max(
        lens[b] for b in range(64) if b not in sharing)
    prefix = tables[sharing[0], :16]
    for b in sharing:
        assert torch.equal(tables[b, :16], prefix)
    private = []
    for b in range(64):
        row = tables[b][tables[b] >= 0]
        assert row.numel() == -(-lens[b] // 256)
        private.extend(row[16:].tolist() if b in sharing else row.tolist())
    assert len(private) == len(set(private)) and not set(private) & set(prefix.tolist())
    unique = sum(lens) - 31 * 4096
    assert w.unique_kv_tokens() == unique
    assert w.algorithmic_bytes() == unique * 2112 + 64 * 32 * 128 * 2 * 2 + 64 * 64 * 4 + 64 * 4


def test_single_sequence_bytes_match_the_stated_figure():
    assert workloads.decode_single("cpu", fill=False).algorithmic_bytes() == 4_341_796
    # Qwen3-VL B=1: 1800 tokens in 8 pages
    assert workloads.decode_qwen_vl("cpu", fill=False).algorithmic_bytes() == 3_818_020


def test_store_and_compaction_workloads():
    s = workloads.store_prefill("cpu")
    assert s.algorithmic_bytes() == 50_888_704
    assert len(set(s.slot_mapping.tolist())) == 8192
    c = workloads.compaction_plans(prefixes=4)
    assert len(c.plans) == 4
    for plan in c.plans:
        assert plan.physical_prompt_len >= 768
        assert not set(plan.source_slots) & set(plan.destination_slots)
    assert c.algorithmic_bytes() == 2 * c.kept * 2112 + 16 * c.kept


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True,
                          text=True, timeout=300, cwd=REPO)
    assert proc.returncode != 0
    assert "one GPU" in proc.stderr
