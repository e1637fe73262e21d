"""GPU parity: seeded random decode configurations against the CPU oracle.

Each seed draws a geometry and a batch:
- kv heads 1, 2, 4 or 8 and GQA groups 1, 2, 4 or 8;
- page sizes 16 to 256;
- batch sizes 1 to 96, with lengths that are ragged, occasionally zero and
  occasionally the table's full capacity;
- holes (-1 block ids) in the tables;
- groups of sequences sharing leading pages.

It runs every kernel family that accepts the geometry (the automatic choice,
the streaming kernel, the per-split kernel) and checks each against
``decode_kernel_semantics`` within the decode tolerance.
"""

from __future__ import annotations

import math

import pytest
import torch

from prism_infer.ops.paged_decode import set_decode_overrides

import oracle
from _helpers import assert_decode_close, require_gpu

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn
MAX_POOL_TOKENS = 96 * 1024


def _config(seed: int, page: int | None = None):
    g = torch.Generator().manual_seed(20261130 + seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=g))]
    hkv = pick([1, 2, 4, 8, 8, 8])
    groups = pick([1, 2, 4, 4, 8])
    drawn = pick([16, 32, 64, 256, 256])
    page = drawn if page is None else page
    batch = int(torch.randint(1, 97, (1,), generator=g))
    max_len = max(1, min(int(torch.randint(1, 12000, (1,), generator=g)), MAX_POOL_TOKENS // batch - page))
    width = math.ceil(max_len / page) + 1
    pool = batch * width + 8
    lens = torch.randint(0, max_len + 1, (batch,), generator=g, dtype=torch.int32)
    lens[torch.rand(batch, generator=g) < 0.08] = 0
    lens[torch.rand(batch, generator=g) < 0.08] = width * page          # the table's full capacity
    tables = torch.randperm(pool, generator=g)[: batch * width].to(torch.int32).view(batch, width).clone()
    tables[torch.rand(batch, width, generator=g) < 0.04] = -1           # holes: skipped tokens
    if batch >= 4 and torch.rand(1, generator=g).item() < 0.6:          # a prefix-sharing group
        members = torch.randperm(batch, generator=g)[: max(2, batch // 3)]
        shared = int(torch.randint(1, max(2, width), (1,), generator=g))
        tables[members, :shared] = tables[members[0], :shared]
    d = 128
    q = torch.randn(batch, hkv * groups, d, generator=g).to(torch.bfloat16)
    src_k = torch.randn(pool, page, hkv, d, generator=g).to(torch.bfloat16)
    src_v = torch.randn(pool, page, hkv, d, generator=g).to(torch.bfloat16)
    return q, src_k, src_v, tables, lens


def _quantize(src):
    n, p, h, d = src.shape
    flat = src.reshape(n * p, h, d)
    k = torch.zeros(n, p, h, d, dtype=FP8)
    s = torch.zeros(n, p, h, dtype=torch.float32)
    oracle.store_scaled(flat, flat, k, torch.zeros_like(k), torch.arange(n * p, dtype=torch.int32), s,
                        torch.zeros_like(s))
    return k, s


@pytest.mark.parametrize("seed,page", [(s, None) for s in range(10)] + [(s, 128) for s in (10, 11, 16, 17, 20, 24, 31)])
def test_random_decode_configs_all_families(seed, page, monkeypatch):
    """Ten random geometries with the page size drawn from {16, 32, 64, 256},
    and seven more at page size 128 (kv heads 1, 2, 4 and 8), a page size the
    reference supports (config.py:46)."""

    require_gpu()
    from prism_infer.ops.paged_decode import paged_decode_attention

    q, src_k, src_v, tables, lens = _config(seed, page)
    k, ks = _quantize(src_k)
    v, vs = _quantize(src_v)
    scale = 128 ** -0.5
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens, scale, k_scale_cache=ks, v_scale_cache=vs,
                                          compute_dtype=torch.float32)
    dev = torch.device("cuda")
    to = lambda t: t.view(torch.uint8).to(dev).view(FP8) if t.dtype == FP8 else t.to(dev)
    args = (to(q), to(k), to(v), to(tables), to(lens), scale)
    kw = dict(k_scale_cache=to(ks), v_scale_cache=to(vs))
    label = f"seed {seed}: B={q.shape[0]} Hq={q.shape[1]} Hkv={k.shape[2]} page={k.shape[1]} W={tables.shape[1]}"
    print(label, flush=True)
    for path in ("auto", "stream", "split"):
        if path == "auto":
            set_decode_overrides(path="auto")
        else:
            set_decode_overrides(path=path)
        got = paged_decode_attention(*args, **kw)
        torch.cuda.synchronize()
        assert_decode_close(got, want, label=f"{label} path={path}")
        assert torch.all(got[lens.to(dev) == 0] == 0), "ctx=0 rows must be zeros"


@pytest.mark.parametrize("batch", [300, 1024, 1030])
def test_large_batches_all_families(batch, monkeypatch):
    """Batches past the prefix-sharing analysis (256), at the streaming path's
    limit (1024) and past it (the per-split path takes over): ragged and zero
    lengths, holes and shared leading pages, on every family that accepts them."""

    require_gpu()
    from prism_infer import _native
    from prism_infer.ops.paged_decode import paged_decode_attention

    g = torch.Generator().manual_seed(20261204 + batch)
    page, width, hkv, groups, d = 16, 8, 8, 4, 128
    pool = batch * width + 8
    lens = torch.randint(0, width * page + 1, (batch,), generator=g, dtype=torch.int32)
    lens[torch.rand(batch, generator=g) < 0.05] = 0
    tables = torch.randperm(pool, generator=g)[: batch * width].to(torch.int32).view(batch, width).clone()
    tables[torch.rand(batch, width, generator=g) < 0.03] = -1
    members = torch.randperm(batch, generator=g)[:64]
    tables[members, :3] = tables[members[0], :3]  # a group sharing three leading pages
    q = torch.randn(batch, hkv * groups, d, generator=g).to(torch.bfloat16)
    k, ks = _quantize(torch.randn(pool, page, hkv, d, generator=g).to(torch.bfloat16))
    v, vs = _quantize(torch.randn(pool, page, hkv, d, generator=g).to(torch.bfloat16))
    scale = d ** -0.5
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens, scale, k_scale_cache=ks, v_scale_cache=vs,
                                          compute_dtype=torch.float32)
    dev = torch.device("cuda")
    to = lambda t: t.view(torch.uint8).to(dev).view(FP8) if t.dtype == FP8 else t.to(dev)
    args = (to(q), to(k), to(v), to(tables), to(lens), scale)
    kw = dict(k_scale_cache=to(ks), v_scale_cache=to(vs))
    family = _native.lib().prism_paged_decode_kernel_family(batch, hkv * groups, hkv, d, page, width, 3)
    print(f"B={batch}: automatic family {family}", flush=True)
    assert family == (2 if batch <= 1024 else 1), "streaming up to 1024 sequences, per-split beyond"
    for path in ("auto", "split") + (("stream",) if batch <= 1024 else ()):
        if path == "auto":
            set_decode_overrides(path="auto")
        else:
            set_decode_overrides(path=path)
        got = paged_decode_attention(*args, **kw)
        torch.cuda.synchronize()
        assert_decode_close(got, want, label=f"B={batch} path={path}")
        assert torch.all(got[lens.to(dev) == 0] == 0), "ctx=0 rows must be zeros"


@pytest.mark.parametrize("hkv,hq", [(4, 16), (4, 32), (2, 8), (2, 16), (1, 8), (1, 16)])
def test_fewer_kv_heads_streaming(hkv, hq, monkeypatch):
    """Four, two or one kv heads (tensor-parallel shards of an 8-head model) on
    the streaming path: two, four or eight tokens per LDS row, as many waves per kv head,
    merged per token slot; a group of sequences sharing two leading pages
    exercises the virtual sequences."""

    require_gpu()
    from prism_infer import _native
    from prism_infer.ops.paged_decode import paged_decode_attention

    g = torch.Generator().manual_seed(20261207 + 100 * hkv + hq)
    batch, page, d = 48, 256, 128
    width = 13
    pool = batch * width + 8
    lens = torch.randint(100, width * page + 1, (batch,), generator=g, dtype=torch.int32)
    lens[:3] = torch.tensor([1, 2, 33], dtype=torch.int32)  # tails shorter than a tile
    lens[5] = 0
    tables = torch.randperm(pool, generator=g)[: batch * width].to(torch.int32).view(batch, width).clone()
    members = torch.arange(10, 26)
    lens[members] = torch.clamp(lens[members], min=2 * page + 1)
    tables[members, :2] = tables[members[0], :2]  # 16 sequences share two leading pages
    tables[40, 4] = -1  # a hole
    q = torch.randn(batch, hq, d, generator=g).to(torch.bfloat16)
    k, ks = _quantize(torch.randn(pool, page, hkv, d, generator=g).to(torch.bfloat16))
    v, vs = _quantize(torch.randn(pool, page, hkv, d, generator=g).to(torch.bfloat16))
    scale = d ** -0.5
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens, scale, k_scale_cache=ks, v_scale_cache=vs,
                                          compute_dtype=torch.float32)
    dev = torch.device("cuda")
    to = lambda t: t.view(torch.uint8).to(dev).view(FP8) if t.dtype == FP8 else t.to(dev)
    args = (to(q), to(k), to(v), to(tables), to(lens), scale)
    kw = dict(k_scale_cache=to(ks), v_scale_cache=to(vs))
    for path in ("stream", "split"):
        set_decode_overrides(path=path)
        # one kv head makes 128-token tiles: this batch is too small for the
        # automatic choice to stream, so the family is checked as forced
        family = _native.lib().prism_paged_decode_kernel_family(batch, hq, hkv, d, page, width, 3)
        assert family == (2 if path == "stream" else 1), (path, family)
        got = paged_decode_attention(*args, **kw)
        torch.cuda.synchronize()
        assert_decode_close(got, want, label=f"Hkv={hkv} Hq={hq} path={path}")
        assert torch.all(got[lens.to(dev) == 0] == 0), "ctx=0 rows must be zeros"


@pytest.mark.parametrize("batch,ctx,family", [(1, 1800, 1), (2, 16384, 1), (2, 32768, 1), (4, 8192, 1),
                                              (4, 16384, 1), (4, 32768, 2), (8, 2048, 1), (8, 4096, 1),
                                              (8, 8192, 2), (16, 512, 1), (16, 1024, 2), (32, 512, 2),
                                              (64, 256, 2), (64, 16384, 2)])
def test_family_choice_by_batch_and_capacity(batch, ctx, family):
    """The automatic family on a 256-CU MI355X (8 kv heads, 256-token pages,
    scaled FP8): the streaming kernel needs enough tiles for the batch (4 per
    workgroup from 16 sequences, 16 from 8, 32 from 4), the per-split kernel
    takes the rest; both give the decode semantics, so this pins speed only."""

    require_gpu()
    from prism_infer import _native

    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("thresholds are stated for 256 compute units")
    set_decode_overrides(path="auto")
    width = -(-ctx // 256)
    got = _native.lib().prism_paged_decode_kernel_family(batch, 32, 8, 128, 256, width,
                                                        _native.dtype_code(torch.float8_e4m3fn))
    assert got == family, (batch, ctx, got)
