"""GPU parity of paged decode over bf16 and f16 KV caches (the dense variants).

A 16-bit cache whose dtype is the query's runs the streaming kernel's 16-bit
tiles (8 kv heads and batches with enough tiles; K rows feed the QK MFMA as
they are, V comes from 16-bit transposed LDS reads) or the split-K kernel (the
K rows feed the QK MFMA as they are; V pairs are assembled with byte
permutes); other 16-bit combinations run the generic kernel.  Each case is compared with
``decode_kernel_semantics`` (the float64 oracle of
prism_infer/ops/paged_decode.py:83-180) within the decode tolerance of
tests/test_scaled_fp8_kv_cache.py:470-472.  The reference's decode reads a
bf16 or f16 cache without scales (``kv_cache_dtype`` auto), as here.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from _helpers import assert_decode_close, require_gpu
from prism_infer.ops.paged_decode import set_decode_overrides

pytestmark = pytest.mark.gpu


def _case(seed, dtype, batch=6, hkv=8, groups=4, page=256, width=12, holes=0.0):
    g = torch.Generator().manual_seed(seed)
    pool = batch * width + 3
    q = torch.randn(batch, hkv * groups, 128, generator=g).to(dtype)
    k = (torch.randn(pool, page, hkv, 128, generator=g) * 2).to(dtype)
    v = torch.randn(pool, page, hkv, 128, generator=g).to(dtype)
    tables = torch.randperm(pool, generator=g)[: batch * width].to(torch.int32).view(batch, width).clone()
    if holes:
        tables[torch.rand(batch, width, generator=g) < holes] = -1
    lens = torch.randint(1, width * page + 1, (batch,), generator=g, dtype=torch.int32)
    lens[0] = width * page
    lens[-1] = 0
    return q, k, v, tables, lens


def _run(q, k, v, tables, lens, scale):
    from prism_infer.ops.paged_decode import paged_decode_attention

    dev = torch.device("cuda")
    out = paged_decode_attention(q.to(dev), k.to(dev), v.to(dev), tables.to(dev), lens.to(dev), scale)
    torch.cuda.synchronize()
    return out.cpu()


def _family(q, k, tables):
    from prism_infer import _native

    return _native.lib().prism_paged_decode_kernel_family(q.shape[0], q.shape[1], k.shape[2], 128, k.shape[1],
                                                          tables.shape[1], _native.dtype_code(k.dtype))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_16bit_cache_split_kernel(dtype):
    require_gpu()
    q, k, v, tables, lens = _case(20261210, dtype, holes=0.05)
    assert _family(q, k, tables) == 1
    scale = 128 ** -0.5
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens, scale)
    for split in (0, 256, 1024):
        set_decode_overrides(path="split", split_tokens=split)
        got = _run(q, k, v, tables, lens, scale)
        assert torch.all(got[-1] == 0)
        assert_decode_close(got, want, label=f"{dtype} split={split}")


@pytest.mark.parametrize("hkv,groups,page", [(4, 4, 64), (2, 8, 48), (1, 16, 256)])
def test_16bit_cache_shapes(hkv, groups, page):
    """Fewer kv heads, page sizes that do not hold whole 32-token tiles, G up to 16."""

    require_gpu()
    q, k, v, tables, lens = _case(20261211 + hkv, torch.bfloat16, batch=3, hkv=hkv, groups=groups, page=page,
                                  width=9)
    scale = 0.07
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens, scale)
    got = _run(q, k, v, tables, lens, scale)
    assert_decode_close(got, want, label=f"bf16 hkv={hkv} G={groups} P={page}")


def test_mixed_16bit_dtypes_use_the_generic_kernel():
    """An f16 query over a bf16 cache (and the reverse) keeps the generic kernel's exact dequantisation."""

    require_gpu()
    q, k, v, tables, lens = _case(20261212, torch.bfloat16, batch=2, width=4)
    scale = 128 ** -0.5
    for qd, kd in ((torch.float16, torch.bfloat16), (torch.bfloat16, torch.float16)):
        qq, kk, vv = q.to(qd), k.to(kd), v.to(kd)
        want = oracle.decode_kernel_semantics(qq, kk, vv, tables, lens, scale)
        got = _run(qq, kk, vv, tables, lens, scale)
        assert_decode_close(got, want, label=f"q {qd} cache {kd}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("page", [256, 64, 16])
def test_16bit_cache_streaming_kernel(dtype, page):
    """The streaming kernel's 16-bit tiles, forced and automatic: ragged lengths (one token, tile tails,
    the table's full capacity, zero), holes, NaN bytes in the pages past every sequence's end (masked
    out, never multiplied), and a group of sequences sharing leading pages (virtual walks)."""

    require_gpu()
    g = torch.Generator().manual_seed(20261213 + page)
    batch, hkv, groups = 40, 8, 4
    width = max(2, 6144 // page)
    pool = batch * width + 5
    q = torch.randn(batch, hkv * groups, 128, generator=g).to(dtype)
    k = (torch.randn(pool, page, hkv, 128, generator=g) * 2).to(dtype)
    v = torch.randn(pool, page, hkv, 128, generator=g).to(dtype)
    tables = torch.randperm(pool, generator=g)[: batch * width].to(torch.int32).view(batch, width).clone()
    lens = torch.randint(1, width * page + 1, (batch,), generator=g, dtype=torch.int32)
    lens[:4] = torch.tensor([1, 15, 17, width * page], dtype=torch.int32)
    lens[5] = 0
    tables[7, 1] = -1
    members = torch.arange(10, 22)
    lens[members] = torch.clamp(lens[members], min=2 * page + 3)
    tables[members, :2] = tables[members[0], :2]
    for b in range(batch):  # garbage past each end: NaN rows in the last page's tail
        n = int(lens[b])
        if 0 < n < width * page and n % page:
            blk = int(tables[b, n // page])
            if blk >= 0:
                k[blk, n % page:] = float("nan")
                v[blk, n % page:] = float("nan")
    scale = 128 ** -0.5
    shared = {int(tables[b, j]) for b in range(batch) for j in range(width) if int(tables[b, j]) >= 0}
    assert len(shared) < batch * width  # the group's pages appear more than once
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens, scale)
    for path in ("stream", "auto"):
        set_decode_overrides(path=path)
        fam = _family(q, k, tables)
        if path == "stream":
            assert fam == 2
        got = _run(q, k, v, tables, lens, scale)
        assert torch.all(got[5] == 0), "ctx = 0 row"
        assert_decode_close(got, want, label=f"{dtype} P={page} path={path} family={fam}")


def test_16bit_cache_streaming_is_automatic_for_large_batches():
    require_gpu()
    q, k, v, tables, lens = _case(20261214, torch.bfloat16, batch=64, width=40)
    assert _family(q, k, tables) == 2
    scale = 128 ** -0.5
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens, scale)
    got = _run(q, k, v, tables, lens, scale)
    assert_decode_close(got, want, label="bf16 B=64 automatic")
