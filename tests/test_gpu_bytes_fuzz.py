"""GPU parity, bit-exact: seeded random KV stores and slot compactions against the CPU oracle.

Store: random token counts, head counts and head dims, bf16 / f16 / f32
inputs, row-strided input views (a packed-QKV layout), 3-D or 4-D caches and
slot mappings with -1 (skipped) entries, with outliers in the data.

Compaction: random source and (unique) destination slot sets drawn from the
same range, so that destinations overwrite other entries' sources (the
staged path) or do not (the one-pass path), on FP8 payload caches and fp32
scale caches of several row widths.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from _helpers import require_gpu

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


@pytest.mark.parametrize("seed", range(8))
def test_random_scaled_store_bit_exact(seed):
    require_gpu()
    from prism_infer.ops.kv_cache_store import store_kvcache

    g = torch.Generator().manual_seed(20261201 + seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=g))]
    heads = pick([1, 2, 4, 8])
    dim = pick([64, 128])
    dtype = pick([torch.bfloat16, torch.float16, torch.float32])
    page = pick([16, 64, 256])
    tokens = int(torch.randint(1, 3000, (1,), generator=g))
    pages = (tokens + page - 1) // page + int(torch.randint(1, 8, (1,), generator=g))
    wide = pick([1, 3])  # 3: K and V are row-strided views of a packed [T, 3, H, D] buffer
    raw = torch.randn(tokens, wide, heads, dim, generator=g)
    raw[torch.rand(raw.shape, generator=g) < 0.01] *= 20.0
    raw = raw.to(dtype)
    key = raw[:, 0]
    value = raw[:, wide - 1] if wide == 1 else raw[:, 1]
    slots = torch.randperm(pages * page, generator=g)[:tokens].to(torch.int32)
    slots[torch.rand(tokens, generator=g) < 0.05] = -1
    three_d = bool(torch.randint(2, (1,), generator=g))
    shape = (pages * page, heads, dim) if three_d else (pages, page, heads, dim)
    sshape = shape[:-1]  # scale caches follow the payload's shape without head_dim
    kc = torch.randint(0, 256, shape, generator=g, dtype=torch.uint8)  # untouched slots keep these bytes
    vc = torch.randint(0, 256, shape, generator=g, dtype=torch.uint8)
    ks = torch.rand(sshape, generator=g)
    vs = torch.rand(sshape, generator=g)

    dev = torch.device("cuda")
    gk, gv = kc.to(dev).view(FP8), vc.to(dev).view(FP8)
    gks, gvs = ks.to(dev), vs.to(dev)
    store_kvcache(key.to(dev), value.to(dev), gk, gv, slots.to(dev), gks, gvs)
    wk, wv, wks, wvs = kc.clone().view(FP8), vc.clone().view(FP8), ks.clone(), vs.clone()
    oracle.store_scaled(key.contiguous(), value.contiguous(), wk, wv, slots, wks, wvs)
    torch.cuda.synchronize()
    label = f"seed {seed}: T={tokens} H={heads} D={dim} {dtype} page={page} wide={wide} 3d={three_d}"
    assert torch.equal(gk.view(torch.uint8).cpu(), wk.view(torch.uint8)), label + ": K bytes"
    assert torch.equal(gv.view(torch.uint8).cpu(), wv.view(torch.uint8)), label + ": V bytes"
    assert torch.equal(gks.cpu().view(torch.int32), wks.view(torch.int32)), label + ": K scales"
    assert torch.equal(gvs.cpu().view(torch.int32), wvs.view(torch.int32)), label + ": V scales"


@pytest.mark.parametrize("seed", range(8))
def test_random_compaction_bit_exact(seed):
    require_gpu()
    from prism_infer.ops.kv_compaction import compact_kv_slots

    g = torch.Generator().manual_seed(20261202 + seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=g))]
    slots = int(torch.randint(64, 20000, (1,), generator=g))
    retained = int(torch.randint(1, max(2, slots // 2), (1,), generator=g))
    layers = pick([1, 2, 3])
    overlap = bool(torch.randint(2, (1,), generator=g))
    src = torch.randint(0, slots, (retained,), generator=g, dtype=torch.long)   # repeats allowed
    if overlap:  # destinations drawn from the whole range: some are other entries' sources
        dst = torch.randperm(slots, generator=g)[:retained]
    else:        # destinations disjoint from every source
        free = torch.ones(slots, dtype=torch.bool)
        free[src] = False
        cand = free.nonzero().flatten()
        dst = cand[torch.randperm(cand.numel(), generator=g)[: min(retained, cand.numel())]]
        src = src[: dst.numel()]
    payload = torch.randint(0, 256, (2, layers, slots, 8, pick([16, 128])), generator=g, dtype=torch.uint8)
    scales = torch.rand(2, layers, slots, 8, generator=g)
    dev = torch.device("cuda")
    label = f"seed {seed}: slots={slots} retained={src.numel()} layers={layers} overlap={overlap}"
    for cache in (payload.view(FP8), scales):
        gpu = cache.view(torch.uint8).to(dev).view(FP8) if cache.dtype == FP8 else cache.to(dev)
        compact_kv_slots(gpu, src.to(dev), dst.to(dev))
        want = cache.clone()
        oracle.compact_slots(want, src, dst)
        torch.cuda.synchronize()
        got = gpu.view(torch.uint8).cpu() if gpu.dtype == FP8 else gpu.cpu()
        want = want.view(torch.uint8) if want.dtype == FP8 else want
        assert torch.equal(got.contiguous().view(torch.uint8), want.contiguous().view(torch.uint8)), label
