"""The drop-in ops' own CPU branch (host tensors), pinned against the oracle.

The reference sends CPU tensors of ``store_kvcache`` to its eager loop
(prism_infer/ops/kv_cache_store.py:439-476, loop :183-230) and CPU caches of
``compact_kv_slots`` to torch index ops (ops/kv_compaction.py:105-112).  This
build's ops do the same work with vectorized torch code of their own; these
tests check it byte for byte against the C oracle (``oracle_store_scaled``,
``oracle_store_unit``, ``oracle_compact_slots``) and against the reference's
per-token loop semantics that the C oracle does not cover (a slot named twice:
the last token wins; an out-of-range slot raises).
"""

from __future__ import annotations

import pytest
import torch

import oracle
from prism_infer.ops.kv_cache_store import store_kvcache
from prism_infer.ops.kv_compaction import compact_kv_slots

FP8 = torch.float8_e4m3fn


def _inputs(tokens, heads, dim, dtype, seed, outliers=True):
    g = torch.Generator().manual_seed(seed)
    key = torch.randn(tokens, heads, dim, generator=g)
    value = torch.randn(tokens, heads, dim, generator=g)
    if outliers:
        mask = torch.rand(tokens, heads, dim, generator=g) < 0.01
        key = torch.where(mask, key * 20, key)
        value = torch.where(mask, value * -20, value)
    return key.to(dtype), value.to(dtype), g


def _bytes(t):
    return t.contiguous().view(torch.uint8)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("cache_rank", [3, 4])
def test_scaled_store_matches_oracle(dtype, cache_rank):
    pages, page, heads, dim = 6, 16, 8, 128
    key, value, g = _inputs(70, heads, dim, dtype, seed=31 + cache_rank)
    slots = torch.randperm(pages * page, generator=g)[:70].to(torch.int32)
    slots[::9] = -1
    shape = (pages, page, heads, dim) if cache_rank == 4 else (pages * page, heads, dim)
    caches = [torch.zeros(shape, dtype=FP8) for _ in range(2)]
    scales = [torch.zeros(shape[:-1]) for _ in range(2)]
    want_c = [c.clone() for c in caches]
    want_s = [s.clone() for s in scales]
    store_kvcache(key, value, *caches, slots, *scales)
    oracle.store_scaled(key, value, *want_c, slots, *want_s)
    for got, want in zip(caches + scales, want_c + want_s):
        assert torch.equal(_bytes(got), _bytes(want))


def test_scaled_store_special_rows():
    """Zero rows (scale floor), a tiny row, a huge row and NaN/inf inputs."""

    heads, dim = 2, 16
    key = torch.randn(5, heads, dim)
    key[0] = 0.0
    key[1] = 1e-9
    key[2, 0] = 3e38
    key[3, 1, 5] = float("nan")
    key[4, 0, 2] = float("inf")
    value = -key
    slots = torch.arange(5, dtype=torch.int32)
    caches = [torch.zeros(8, heads, dim, dtype=FP8) for _ in range(2)]
    scales = [torch.zeros(8, heads) for _ in range(2)]
    want_c = [c.clone() for c in caches]
    want_s = [s.clone() for s in scales]
    store_kvcache(key, value, *caches, slots, *scales)
    oracle.store_scaled(key, value, *want_c, slots, *want_s)
    for got, want in zip(caches + scales, want_c + want_s):
        assert torch.equal(_bytes(got), _bytes(want))


def test_unit_scale_and_dense_store():
    heads, dim = 4, 32
    key, value, g = _inputs(40, heads, dim, torch.bfloat16, seed=5, outliers=False)
    slots = torch.randperm(64, generator=g)[:40].to(torch.int32)
    slots[3] = -1
    kc = torch.zeros(64, heads, dim, dtype=FP8)
    vc = torch.zeros_like(kc)
    wk, wv = kc.clone(), vc.clone()
    store_kvcache(key, value, kc, vc, slots)
    oracle.store_unit(key, value, wk, wv, slots)
    assert torch.equal(_bytes(kc), _bytes(wk)) and torch.equal(_bytes(vc), _bytes(wv))

    dense_k = torch.zeros(4, 16, heads, dim, dtype=torch.bfloat16)
    dense_v = torch.zeros_like(dense_k)
    store_kvcache(key, value, dense_k, dense_v, slots)
    flat = dense_k.view(-1, heads, dim)
    live = slots >= 0
    assert torch.equal(flat[slots[live].long()], key[live])
    untouched = torch.ones(64, dtype=torch.bool)
    untouched[slots[live].long()] = False
    assert bool((flat[untouched] == 0).all())


def test_repeated_slot_keeps_the_last_token():
    """The reference loop writes tokens in order: the last writer of a slot wins."""

    heads, dim = 2, 16
    key, value, _ = _inputs(6, heads, dim, torch.bfloat16, seed=9, outliers=False)
    slots = torch.tensor([3, 1, 3, -1, 1, 3], dtype=torch.int32)
    caches = [torch.zeros(8, heads, dim, dtype=FP8) for _ in range(2)]
    scales = [torch.zeros(8, heads) for _ in range(2)]
    store_kvcache(key, value, *caches, slots, *scales)
    for token in (5, 4):  # last writers of slots 3 and 1
        slot = int(slots[token])
        want_c = [torch.zeros(1, heads, dim, dtype=FP8) for _ in range(2)]
        want_s = [torch.zeros(1, heads) for _ in range(2)]
        oracle.store_scaled(key[token:token + 1], value[token:token + 1], *want_c,
                            torch.zeros(1, dtype=torch.int32), *want_s)
        assert torch.equal(_bytes(caches[0][slot]), _bytes(want_c[0][0]))
        assert torch.equal(_bytes(scales[1][slot]), _bytes(want_s[1][0]))


def test_store_out_of_range_slot_raises_index_error():
    key, value, _ = _inputs(2, 2, 16, torch.float32, seed=1)
    caches = [torch.zeros(4, 2, 16, dtype=FP8) for _ in range(2)]
    scales = [torch.zeros(4, 2) for _ in range(2)]
    with pytest.raises(IndexError):
        store_kvcache(key, value, *caches, torch.tensor([0, 4], dtype=torch.int32), *scales)


@pytest.mark.parametrize("pattern", ["shift", "swap", "cycle", "random"])
@pytest.mark.parametrize("scales", [False, True])
def test_compaction_matches_oracle(pattern, scales):
    g = torch.Generator().manual_seed(77)
    slots = 96
    shape = (2, 3, slots, 4) if scales else (2, 3, slots, 4, 32)
    if scales:
        cache = torch.randn(shape, generator=g)
    else:
        cache = torch.randint(0, 256, shape, generator=g, dtype=torch.uint8).view(FP8)
    if pattern == "shift":
        src = torch.arange(10, 60)
        dst = src - 7
    elif pattern == "swap":
        src = torch.tensor([5, 40, 6, 41])
        dst = torch.tensor([40, 5, 41, 6])
    elif pattern == "cycle":
        src = torch.tensor([1, 2, 3, 4])
        dst = torch.tensor([2, 3, 4, 1])
    else:
        src = torch.randperm(slots, generator=g)[:50]
        dst = torch.randperm(slots, generator=g)[:50]
    want = cache.clone()
    compact_kv_slots(cache, src, dst)
    oracle.compact_slots(want, src, dst)
    assert torch.equal(_bytes(cache), _bytes(want))


def test_compaction_out_of_range_raises():
    """torch's index_select raises for an out-of-range slot, as in the reference."""

    cache = torch.zeros(2, 1, 16, 2, 8, dtype=FP8)
    with pytest.raises((IndexError, RuntimeError), match="out of"):
        compact_kv_slots(cache, torch.tensor([1, 16]), torch.tensor([0, 1]))
