"""CPU tests: uniform visual-token retention (the policy in front of compaction).

Known answers come from the reference's tests and from hand computation of
the rule "ordinal round(k (n-1) / (t-1)), ties to even"; the remaining checks
are properties the rule fixes (endpoints, count, spacing) and the
composition with the in-place compaction plan.
"""

from __future__ import annotations

import pytest

from prism_infer.engine.kv_compaction_plan import plan_in_place
from prism_infer.engine.visual_pruning import retained_positions, target_keep_count, uniform_keep_indices


def test_reference_known_answers():
    # test_visual_pruning.py:46-60: visual tokens at 1, 2, 4, 5, 7; ratio 0.4, floor 1
    visual = (1, 2, 4, 5, 7)
    t = target_keep_count(len(visual), min_keep_tokens=1, keep_ratio=0.4)
    assert t == 2
    assert uniform_keep_indices(visual, t) == (1, 7)
    # test_visual_pruning.py:69-100: 10 tokens at ratio 0.5, floors 8 and 2
    assert target_keep_count(10, min_keep_tokens=8, keep_ratio=0.5) == 8
    assert target_keep_count(10, min_keep_tokens=2, keep_ratio=0.5) == 5


@pytest.mark.parametrize("n,t,want", [
    (10, 4, (0, 3, 6, 9)),        # spacing 3
    (6, 4, (0, 2, 3, 5)),         # 5/3: 1.67 -> 2, 3.33 -> 3
    (12, 5, (0, 3, 6, 8, 11)),    # 2.75: 5.5 -> 6 (even)
    (10, 3, (0, 4, 9)),           # 4.5 -> 4 (even), not 5
    (6, 3, (0, 2, 5)),            # 2.5 -> 2 (even), not 3
    (8, 3, (0, 4, 7)),            # 3.5 -> 4 (even)
    (4, 3, (0, 2, 3)),            # 1.5 -> 2 (even)
    (7, 1, (3,)),                 # one keep: the middle
    (8, 1, (4,)),
    (5, 5, (0, 1, 2, 3, 4)),      # all kept
    (5, 9, (0, 1, 2, 3, 4)),
    (5, 0, ()),
])
def test_hand_computed_ordinals(n, t, want):
    assert uniform_keep_indices(range(n), t) == want
    # ordinals index the given token positions
    offset = tuple(100 + 3 * i for i in range(n))
    assert uniform_keep_indices(offset, t) == tuple(offset[o] for o in want)


@pytest.mark.parametrize("n", [2, 3, 17, 196, 1000, 8128])
def test_properties(n):
    for t in sorted({2, 3, n // 3 + 1, (n + 1) // 2, n - 1, n} - {0, 1}):
        keep = uniform_keep_indices(range(n), t)
        assert len(keep) == min(t, n)
        assert keep[0] == 0 and keep[-1] == n - 1
        assert list(keep) == sorted(set(keep))
        if t < n:
            spacing = (n - 1) / (t - 1)
            gaps = {b - a for a, b in zip(keep, keep[1:])}
            assert gaps <= {int(spacing), int(spacing) + 1}, (n, t, gaps)


def test_target_keep_count_edges():
    assert target_keep_count(0) == 0
    assert target_keep_count(-3) == 0
    assert target_keep_count(20) == 20            # at or under the default floor of 32
    assert target_keep_count(32) == 32
    assert target_keep_count(33) == 32            # ceil(19.8) = 20 < floor
    assert target_keep_count(100) == 60           # default ratio 0.6
    assert target_keep_count(8128) == 4877        # ceil(4876.8)
    assert target_keep_count(8128, min_keep_tokens=768, keep_ratio=0.05) == 768
    assert target_keep_count(10, min_keep_tokens=4, keep_ratio=2.0) == 10


def test_retained_positions_feed_the_in_place_plan():
    # a prompt of 4 pages: 64 text tokens, 8128 visual positions [64, 8192)
    page = 256
    prompt = 4 * page
    visual = tuple(range(64, prompt))
    kept = retained_positions(prompt, visual, min_keep_tokens=32, keep_ratio=0.6)
    n_keep = target_keep_count(len(visual), min_keep_tokens=32, keep_ratio=0.6)
    assert len(kept) == 64 + n_keep
    assert kept[:64] == tuple(range(64))
    assert set(kept[64:]) == set(uniform_keep_indices(visual, n_keep))
    plan = plan_in_place((7, 3, 9, 1), kept, page, logical_prompt_len=prompt, compacted_logical_len=prompt)
    assert len(plan.source_slots) == len(kept)
    # the retained token at rank i moves to slot i of the kept page prefix
    assert plan.source_slots[:64] == tuple(7 * page + p for p in range(64))
    assert plan.destination_slots[0] == 7 * page and plan.destination_slots[-1] == \
        (7, 3, 9, 1)[(len(kept) - 1) // page] * page + (len(kept) - 1) % page


def test_retained_positions_rejects_bad_indices():
    with pytest.raises(ValueError):
        retained_positions(10, (3, 10))
    with pytest.raises(ValueError):
        retained_positions(10, (3, 3))
