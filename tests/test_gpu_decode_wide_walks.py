"""GPU parity: virtual walks of shared pages with two query-column blocks.

On tiles of 8 kv heads (scaled FP8, or a bf16/f16 cache of the query's
dtype) the streaming kernel walks a group's shared
leading pages once for 32 / G members (two 16-column MFMA blocks per walk);
with fewer kv heads a walk keeps one block of 16 columns.  These cases put
groups of 2, 3, 8, 9, 17 and 33 sharers (more than one walk's worth, a
remainder of one member, which is not a walk, and partial last pages) next to
private sequences, for G = 1, 2, 3, 4, 6, 8 and 16 (with G = 3 and 6 the 32
columns hold 10 and 5 members and two columns stay empty), and check the
streaming kernel against ``decode_kernel_semantics`` within the decode
tolerance, and that a second call on the same plan gives the same bits.
"""

from __future__ import annotations

import pytest
import torch

from prism_infer.ops.paged_decode import set_decode_overrides

import oracle
from _helpers import assert_decode_close, require_gpu

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn
GROUP_SIZES = (2, 3, 8, 9, 17, 33)


def _quantize(src):
    n, p, h, d = src.shape
    flat = src.reshape(n * p, h, d)
    k = torch.zeros(n, p, h, d, dtype=FP8)
    s = torch.zeros(n, p, h, dtype=torch.float32)
    oracle.store_scaled(flat, flat, k, torch.zeros_like(k), torch.arange(n * p, dtype=torch.int32), s,
                        torch.zeros_like(s))
    return k, s


def _batch(hkv: int, groups: int, seed: int, dtype=None):
    g = torch.Generator().manual_seed(20261202 + 97 * hkv + groups + seed)
    page, width, d = 64, 12, 128
    private = 16
    batch = sum(GROUP_SIZES) + private
    pool = batch * width + 8
    tables = torch.randperm(pool, generator=g)[: batch * width].to(torch.int32).view(batch, width).clone()
    lens = torch.randint(page, width * page + 1, (batch,), generator=g, dtype=torch.int32)
    order = torch.randperm(batch, generator=g)  # group members scattered through the batch
    at = 0
    for size in GROUP_SIZES:
        members = order[at:at + size]
        at += size
        shared = int(torch.randint(1, width - 1, (1,), generator=g))
        tables[members, :shared] = tables[members[0], :shared]
        # some members end inside the shared prefix, one exactly at its end
        lens[members[1]] = shared * page
        lens[members[-1]] = max(1, shared * page - int(torch.randint(1, page, (1,), generator=g)))
    q = torch.randn(batch, hkv * groups, d, generator=g).to(dtype or torch.bfloat16)
    if dtype is not None:  # a 16-bit cache of the query's dtype, no scales
        k = torch.randn(pool, page, hkv, d, generator=g).to(dtype)
        v = torch.randn(pool, page, hkv, d, generator=g).to(dtype)
        return q, k, v, None, None, tables, lens
    k, ks = _quantize(torch.randn(pool, page, hkv, d, generator=g).to(torch.bfloat16))
    v, vs = _quantize(torch.randn(pool, page, hkv, d, generator=g).to(torch.bfloat16))
    return q, k, v, ks, vs, tables, lens


@pytest.mark.parametrize("hkv,groups", [(8, 1), (8, 2), (8, 3), (8, 4), (8, 6), (8, 8), (8, 16), (4, 4), (2, 8)])
def test_shared_prefix_groups_on_the_streaming_kernel(hkv, groups):
    require_gpu()
    from prism_infer.ops.paged_decode import paged_decode_attention

    q, k, v, ks, vs, tables, lens = _batch(hkv, groups, 0)
    scale = 128 ** -0.5
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens, scale, k_scale_cache=ks, v_scale_cache=vs,
                                          compute_dtype=torch.float32)
    dev = torch.device("cuda")
    to = lambda t: t.view(torch.uint8).to(dev).view(FP8) if t.dtype == FP8 else t.to(dev)
    args = (to(q), to(k), to(v), to(tables), to(lens), scale)
    kw = dict(k_scale_cache=to(ks), v_scale_cache=to(vs))
    label = f"B={q.shape[0]} Hq={q.shape[1]} Hkv={hkv} G={groups} groups {GROUP_SIZES}"
    print(label, flush=True)
    set_decode_overrides(path="stream")
    first = paged_decode_attention(*args, **kw)
    again = paged_decode_attention(*args, **kw)
    torch.cuda.synchronize()
    assert_decode_close(first, want, label=label)
    assert torch.equal(first, again), f"{label}: a second call on the same plan differs"


@pytest.mark.parametrize("groups,dtype", [(1, torch.bfloat16), (4, torch.bfloat16), (16, torch.bfloat16),
                                          (3, torch.float16)])
def test_shared_prefix_groups_on_16bit_tiles(groups, dtype):
    """The same groups over a 16-bit cache (two-block walks of 16-bit tiles)."""

    require_gpu()
    from prism_infer.ops.paged_decode import paged_decode_attention

    q, k, v, _, _, tables, lens = _batch(8, groups, 1, dtype)
    scale = 128 ** -0.5
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens, scale, compute_dtype=torch.float32)
    dev = torch.device("cuda")
    args = (q.to(dev), k.to(dev), v.to(dev), tables.to(dev), lens.to(dev), scale)
    label = f"B={q.shape[0]} Hq={q.shape[1]} Hkv=8 G={groups} {dtype} groups {GROUP_SIZES}"
    print(label, flush=True)
    set_decode_overrides(path="stream")
    first = paged_decode_attention(*args)
    again = paged_decode_attention(*args)
    torch.cuda.synchronize()
    assert_decode_close(first, want, label=label)
    assert torch.equal(first, again), f"{label}: a second call on the same plan differs"
