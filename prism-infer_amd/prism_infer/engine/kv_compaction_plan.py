"""Slot mapping for physical KV compaction (host side).

Restates the slot arithmetic of
prism_infer/engine/kv_compaction_coordinator.py:60-92 and the checks of
prism_infer/engine/kv_layout.py:214-263 for the producer of
``compact_kv_slots``' ``source_slots`` / ``destination_slots``:

    src_i = old_table[pos_i // P] * P + pos_i % P     (pos sorted, unique)
    dst_i = new_table[i // P] * P + i % P

In the reference the new table is the prefix ``old_table[:ceil(final_len/P)]``
(in place, so sources and destinations overlap); :func:`plan_out_of_place`
writes into freshly supplied pages instead (disjoint sets, one-pass copy).
Which tokens to keep is the caller's decision (a keep-mask / position list).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class CompactionSlots:
    source_slots: tuple[int, ...]
    destination_slots: tuple[int, ...]
    new_block_table: tuple[int, ...]
    released_block_ids: tuple[int, ...]
    physical_prompt_len: int
    final_physical_prompt_len: int

    def tensors(self, device: torch.device | str) -> tuple[torch.Tensor, torch.Tensor]:
        """int64 device tensors, as ``compact_kv_slots`` expects."""

        src = torch.tensor(self.source_slots, dtype=torch.long, device=device)
        dst = torch.tensor(self.destination_slots, dtype=torch.long, device=device)
        return src, dst


def _check_positions(retained_positions, compacted_logical_len: int) -> tuple[int, ...]:
    positions = tuple(int(p) for p in retained_positions)
    if not positions:
        raise RuntimeError("visual KV compaction retained zero prompt tokens")
    if tuple(sorted(set(positions))) != positions:
        raise ValueError("plan retained positions must be sorted and unique")
    if positions[0] < 0 or positions[-1] >= compacted_logical_len:
        raise ValueError("plan retained positions exceed compacted prefix")
    return positions


def plan_in_place(old_block_table, retained_positions, block_size: int, *, logical_prompt_len: int,
                  compacted_logical_len: int | None = None) -> CompactionSlots:
    """The reference's plan: compact into the existing page-table prefix."""

    if block_size <= 0:
        raise ValueError(f"block_size must be positive, got {block_size}")
    compacted = logical_prompt_len if compacted_logical_len is None else compacted_logical_len
    if not 1 <= compacted <= logical_prompt_len:
        raise ValueError("compacted logical prefix is outside prompt bounds")
    old = tuple(int(b) for b in old_block_table)
    if len(old) * block_size < logical_prompt_len:
        raise RuntimeError("visual KV compaction requires a complete prompt block table")
    positions = _check_positions(retained_positions, compacted)
    physical = len(positions)
    final_len = physical + (logical_prompt_len - compacted)
    new_blocks = (final_len + block_size - 1) // block_size
    new_table = old[:new_blocks]
    source = tuple(old[p // block_size] * block_size + p % block_size for p in positions)
    destination = tuple(new_table[i // block_size] * block_size + i % block_size for i in range(physical))
    return CompactionSlots(source, destination, new_table, old[new_blocks:], physical, final_len)


def plan_out_of_place(old_block_table, retained_positions, block_size: int, destination_block_table) -> CompactionSlots:
    """Gather the retained tokens into new dense pages ``destination_block_table``."""

    if block_size <= 0:
        raise ValueError(f"block_size must be positive, got {block_size}")
    old = tuple(int(b) for b in old_block_table)
    positions = _check_positions(retained_positions, len(old) * block_size)
    physical = len(positions)
    need = (physical + block_size - 1) // block_size
    dest = tuple(int(b) for b in destination_block_table)
    if len(dest) < need:
        raise ValueError(f"destination table has {len(dest)} pages, {need} needed")
    if set(dest[:need]) & set(old):
        raise ValueError("out-of-place destination pages must not overlap the source pages")
    source = tuple(old[p // block_size] * block_size + p % block_size for p in positions)
    destination = tuple(dest[i // block_size] * block_size + i % block_size for i in range(physical))
    return CompactionSlots(source, destination, dest[:need], old, physical, physical)


__all__ = ["CompactionSlots", "plan_in_place", "plan_out_of_place"]
