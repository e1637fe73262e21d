"""Slot mapping for physical KV compaction (host side).

Restates the slot arithmetic of
prism_infer/engine/kv_compaction_coordinator.py:60-98 and the plan checks of
prism_infer/engine/kv_layout.py:214-263 for the producer of
``compact_kv_slots``' ``source_slots`` / ``destination_slots``:

    src_i = old_table[pos_i // P] * P + pos_i % P     (pos sorted, unique)
    dst_i = new_table[i // P] * P + i % P

In the reference the new table is the prefix ``old_table[:ceil(final_len/P)]``
(in place, so sources and destinations overlap); :func:`plan_out_of_place`
writes into freshly supplied pages instead (disjoint sets, one-pass copy).
Which tokens to keep is the caller's decision (a keep-mask / position list).

Safety contract (kv_compaction_coordinator.py:49-58): an in-place plan rewrites
the sequence's own pages, so it refuses any page another sequence also
references. The caller supplies the reference counts (``ref_counts``: a mapping
or a callable ``block_id -> count``); a count other than 1 raises. The copy
kernel itself has no notion of ownership.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Mapping, Optional, Union

import torch

RefCounts = Union[Mapping[int, int], Callable[[int], int], None]


@dataclass(frozen=True)
class CompactionSlots:
    source_slots: tuple[int, ...]
    destination_slots: tuple[int, ...]
    new_block_table: tuple[int, ...]
    released_block_ids: tuple[int, ...]
    physical_prompt_len: int
    final_physical_prompt_len: int
    old_block_table: tuple[int, ...] = ()
    retained_positions: tuple[int, ...] = ()
    logical_prompt_len: int = 0
    compacted_logical_len: int = 0
    in_place: bool = True

    def tensors(self, device: torch.device | str) -> tuple[torch.Tensor, torch.Tensor]:
        """int64 device tensors, as ``compact_kv_slots`` expects."""

        src = torch.tensor(self.source_slots, dtype=torch.long, device=device)
        dst = torch.tensor(self.destination_slots, dtype=torch.long, device=device)
        return src, dst

    def validate(self, block_size: int) -> None:
        """Re-derive the plan from its own fields and raise on any inconsistency.

        Follows KVCompactionPlan.validate (kv_layout.py:214-263): lengths,
        sorted unique positions inside the compacted prefix, the new table as
        the old table's prefix with the suffix released (in place) and the
        destinations as the dense run of the new table's slots. Source slots
        are checked against the position arithmetic too.
        """

        _check_block_size(block_size)
        n = self.physical_prompt_len
        if not 1 <= self.compacted_logical_len <= self.logical_prompt_len:
            raise ValueError("compacted logical prefix is outside prompt bounds")
        if n != len(self.retained_positions):
            raise ValueError("physical prompt length must equal retained positions")
        if n != len(self.source_slots):
            raise ValueError("physical prompt length must equal source slots")
        if n != len(self.destination_slots):
            raise ValueError("physical prompt length must equal destination slots")
        _check_positions(self.retained_positions, self.compacted_logical_len)
        old, new = self.old_block_table, self.new_block_table
        pages = -(-self.final_physical_prompt_len // block_size)
        if len(new) != pages:
            raise ValueError("plan compact block count is inconsistent")
        if self.in_place:
            if old[:pages] != new:
                raise ValueError("plan must compact into the existing page-table prefix")
            if old[pages:] != self.released_block_ids:
                raise ValueError("plan released blocks must be the old page-table suffix")
        if self.source_slots != _slots_of(old, self.retained_positions, block_size):
            raise ValueError("plan source slots do not follow the retained positions")
        if self.destination_slots != _slots_of(new, range(n), block_size):
            raise ValueError("plan destination slots are not a dense physical tail")


def _check_block_size(block_size: int) -> None:
    if block_size <= 0:
        raise ValueError(f"block_size must be positive, got {block_size}")


def _check_positions(retained_positions, compacted_logical_len: int) -> tuple[int, ...]:
    positions = tuple(int(p) for p in retained_positions)
    if not positions:
        raise RuntimeError("visual KV compaction retained zero prompt tokens")
    if tuple(sorted(set(positions))) != positions:
        raise ValueError("plan retained positions must be sorted and unique")
    if positions[0] < 0 or positions[-1] >= compacted_logical_len:
        raise ValueError("plan retained positions exceed compacted prefix")
    return positions


def _check_table(table: tuple[int, ...], what: str) -> None:
    if any(b < 0 for b in table):
        raise ValueError(f"{what} holds a negative block id: {list(table)}")
    if len(set(table)) != len(table):
        raise ValueError(f"{what} names a block twice: {list(table)}")


def _ref_count(ref_counts: RefCounts, block_id: int) -> int:
    if callable(ref_counts):
        return int(ref_counts(block_id))
    return int(ref_counts[block_id])


def _refuse_shared(table: tuple[int, ...], ref_counts: RefCounts) -> None:
    if ref_counts is None:
        return
    shared = [b for b in table if _ref_count(ref_counts, b) != 1]
    if shared:
        raise RuntimeError("visual KV compaction does not mutate prefix-shared blocks; "
                           f"shared_block_ids={shared}")


def _slots_of(table, positions, block_size: int) -> tuple[int, ...]:
    return tuple(table[p // block_size] * block_size + p % block_size for p in positions)


def plan_in_place(old_block_table, retained_positions, block_size: int, *, logical_prompt_len: int,
                  compacted_logical_len: Optional[int] = None,
                  ref_counts: RefCounts = None) -> CompactionSlots:
    """The reference's plan: compact into the existing page-table prefix.

    ``ref_counts`` (mapping or callable) gives each page's reference count; a
    page held by more than this sequence (count != 1) is refused with the
    reference's RuntimeError, since rewriting it in place would corrupt the
    other holders' KV. Without it the caller vouches that the pages are
    private.
    """

    _check_block_size(block_size)
    compacted = logical_prompt_len if compacted_logical_len is None else compacted_logical_len
    if not 1 <= compacted <= logical_prompt_len:
        raise ValueError("compacted logical prefix is outside prompt bounds")
    old = tuple(int(b) for b in old_block_table)
    if len(old) * block_size < logical_prompt_len:
        raise RuntimeError("visual KV compaction requires a complete prompt block table")
    _check_table(old, "old block table")
    _refuse_shared(old, ref_counts)
    positions = _check_positions(retained_positions, compacted)
    physical = len(positions)
    final_len = physical + (logical_prompt_len - compacted)
    new_blocks = -(-final_len // block_size)
    new_table = old[:new_blocks]
    plan = CompactionSlots(
        source_slots=_slots_of(old, positions, block_size),
        destination_slots=_slots_of(new_table, range(physical), block_size),
        new_block_table=new_table, released_block_ids=old[new_blocks:],
        physical_prompt_len=physical, final_physical_prompt_len=final_len,
        old_block_table=old, retained_positions=positions,
        logical_prompt_len=logical_prompt_len, compacted_logical_len=compacted, in_place=True)
    plan.validate(block_size)
    return plan


def plan_out_of_place(old_block_table, retained_positions, block_size: int,
                      destination_block_table) -> CompactionSlots:
    """Gather the retained tokens into new dense pages ``destination_block_table``.

    The old pages are only read, so shared pages are allowed; the destination
    pages must be distinct from each other and from the old ones.
    """

    _check_block_size(block_size)
    old = tuple(int(b) for b in old_block_table)
    _check_table(old, "old block table")
    logical = len(old) * block_size
    positions = _check_positions(retained_positions, logical)
    physical = len(positions)
    need = -(-physical // block_size)
    dest = tuple(int(b) for b in destination_block_table)
    if len(dest) < need:
        raise ValueError(f"destination table has {len(dest)} pages, {need} needed")
    _check_table(dest[:need], "destination block table")
    if set(dest[:need]) & set(old):
        raise ValueError("out-of-place destination pages must not overlap the source pages")
    plan = CompactionSlots(
        source_slots=_slots_of(old, positions, block_size),
        destination_slots=_slots_of(dest, range(physical), block_size),
        new_block_table=dest[:need], released_block_ids=old,
        physical_prompt_len=physical, final_physical_prompt_len=physical,
        old_block_table=old, retained_positions=positions,
        logical_prompt_len=logical, compacted_logical_len=logical, in_place=False)
    plan.validate(block_size)
    return plan


__all__ = ["CompactionSlots", "plan_in_place", "plan_out_of_place"]
