"""Uniform visual-token retention: which prompt positions a compaction keeps.

Host policy in front of :func:`prism_infer.ops.kv_compaction.compact_kv_slots`:
the kept positions feed :func:`prism_infer.engine.kv_compaction_plan.plan_in_place`
or ``plan_out_of_place``, whose slot lists the kernel moves.

Restates the reference's uniform strategy:

* ``target_keep_count`` follows ``_target_keep_count``
  (``prism_infer/engine/visual_pruning.py:395-407``);
* ``uniform_keep_indices`` follows ``_uniform_keep_indices`` (``:410-435``):
  keep ordinal ``round(k * (n - 1) / (t - 1))`` for k = 0 .. t - 1, with Python's
  ties-to-even rounding, a single keep taking the middle token, and, should
  ordinals coincide, the lowest unused ordinals filling up to ``t``.  The
  rounding here is done on integers (quotient and remainder of
  ``k * (n - 1)`` by ``t - 1``), which gives the nearest integer with ties to
  even exactly, for any size;
* defaults ratio 0.6 and floor 32 are the reference's
  (``visual_pruning.py:21-22``).
"""

from __future__ import annotations

import math
from collections.abc import Sequence

DEFAULT_KEEP_RATIO = 0.6
DEFAULT_MIN_KEEP_TOKENS = 32

__all__ = [
    "DEFAULT_KEEP_RATIO",
    "DEFAULT_MIN_KEEP_TOKENS",
    "retained_positions",
    "target_keep_count",
    "uniform_keep_indices",
]


def target_keep_count(total_visual_tokens: int, *, min_keep_tokens: int = DEFAULT_MIN_KEEP_TOKENS,
                      keep_ratio: float = DEFAULT_KEEP_RATIO) -> int:
    """Visual tokens to keep: all of them up to the floor, else max(floor, ceil(n * ratio)), at most n."""

    n = int(total_visual_tokens)
    if n <= 0:
        return 0
    if n <= min_keep_tokens:
        return n
    return min(n, max(int(min_keep_tokens), math.ceil(n * keep_ratio)))


def _round_ratio_half_even(num: int, den: int) -> int:
    """Nearest integer to num / den (num >= 0, den > 0), ties to the even one."""

    q, r = divmod(num, den)
    twice = 2 * r
    if twice > den or (twice == den and q % 2 == 1):
        return q + 1
    return q


def uniform_keep_indices(visual_token_indices: Sequence[int], target_keep: int) -> tuple[int, ...]:
    """``target_keep`` of the given token indices, spread evenly, in ascending ordinal order."""

    indices = tuple(int(i) for i in visual_token_indices)
    n = len(indices)
    t = int(target_keep)
    if t >= n:
        return indices
    if t <= 0:
        return ()
    if t == 1:
        return (indices[n // 2],)
    chosen: list[int] = []
    seen: set[int] = set()
    for k in range(t):
        o = _round_ratio_half_even(k * (n - 1), t - 1)
        if o not in seen:
            seen.add(o)
            chosen.append(o)
    o = 0
    while len(chosen) < t:  # only if ordinals coincided: lowest unused ones
        if o not in seen:
            seen.add(o)
            chosen.append(o)
        o += 1
    return tuple(indices[o] for o in sorted(chosen))


def retained_positions(prompt_len: int, visual_token_indices: Sequence[int], *,
                       min_keep_tokens: int = DEFAULT_MIN_KEEP_TOKENS,
                       keep_ratio: float = DEFAULT_KEEP_RATIO) -> tuple[int, ...]:
    """Sorted prompt positions a uniform pruning keeps: every non-visual position plus the kept visual ones."""

    visual = tuple(int(i) for i in visual_token_indices)
    if any(i < 0 or i >= prompt_len for i in visual):
        raise ValueError(f"visual token indices must lie in [0, {prompt_len})")
    if len(set(visual)) != len(visual):
        raise ValueError("visual token indices must be unique")
    keep = uniform_keep_indices(visual, target_keep_count(len(visual), min_keep_tokens=min_keep_tokens,
                                                          keep_ratio=keep_ratio))
    dropped = set(visual) - set(keep)
    return tuple(p for p in range(prompt_len) if p not in dropped)
