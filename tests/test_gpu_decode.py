"""GPU parity: HIP paged decode against the CPU oracle (tolerance 2e-2 abs / 1e-2 rel, bf16)."""

from __future__ import annotations

import math

import pytest
import torch

from prism_infer.ops.paged_decode import set_decode_overrides

import oracle
from _helpers import assert_decode_close, compact_to_cpu, require_gpu

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


@pytest.fixture(params=["auto", "stream", "split"])
def decode_path(request, monkeypatch):
    """Run a test with the default kernel choice and with each family forced."""

    if request.param != "auto":
        set_decode_overrides(path=request.param)
    return request.param


def _quantize_cpu(source: torch.Tensor):
    """Scaled-FP8 pages of ``source`` [N, P, H, D] through the oracle."""

    n, p, h, d = source.shape
    flat = source.reshape(n * p, h, d)
    k = torch.zeros(n, p, h, d, dtype=FP8)
    s = torch.zeros(n, p, h, dtype=torch.float32)
    k2 = torch.zeros_like(k)
    s2 = torch.zeros_like(s)
    oracle.store_scaled(flat, flat, k, k2, torch.arange(n * p, dtype=torch.int32), s, s2)
    return k, s


def _decode_gpu(q, k, v, ks, vs, tables, lens, scale, max_ctx=None):
    from prism_infer.ops.paged_decode import paged_decode_attention

    dev = torch.device("cuda")
    to = lambda t: None if t is None else (t.view(torch.uint8).to(dev).view(FP8) if t.dtype == FP8 else t.to(dev))
    out = paged_decode_attention(
        to(q), to(k), to(v), to(tables), to(lens), scale,
        k_scale_cache=to(ks), v_scale_cache=to(vs),
        max_context_len=None if max_ctx is None else torch.tensor([max_ctx], dtype=torch.int32, device=dev),
    )
    torch.cuda.synchronize()
    return out.cpu()


def _oracle(q, k, v, ks, vs, tables, lens, scale, max_ctx=None):
    return oracle.decode_kernel_semantics(q, k, v, tables, lens, scale, k_scale_cache=ks, v_scale_cache=vs,
                                          max_context_len=max_ctx)


def test_reference_scaled_decode_case_seed_20260720():
    """The reference's scaled decode case: B=2, 8q/2kv heads, D=128, 16-token pages, ctx 17/33."""

    require_gpu()
    g = torch.Generator().manual_seed(20260720)
    q = torch.randn(2, 8, 128, generator=g).to(torch.bfloat16)
    k_src = (torch.randn(6, 16, 2, 128, generator=g) * 23.0).to(torch.bfloat16)
    v_src = (torch.randn(6, 16, 2, 128, generator=g) * 15.0).to(torch.bfloat16)
    k, ks = _quantize_cpu(k_src)
    v, vs = _quantize_cpu(v_src)
    tables = torch.arange(6, dtype=torch.int32).view(2, 3)
    lens = torch.tensor([17, 33], dtype=torch.int32)
    got = _decode_gpu(q, k, v, ks, vs, tables, lens, 128 ** -0.5)
    want = oracle.decode_reference_fp32(q, k, v, ks, vs, tables, lens, 128 ** -0.5)
    assert_decode_close(got, want, label="ref-20260720")
    assert_decode_close(got, _oracle(q, k, v, ks, vs, tables, lens, 128 ** -0.5), label="ref-20260720-f64")


@pytest.mark.parametrize("batch", [1, 2, 4, 8])
def test_qwen_batch_context_matrix_scaled_fp8(batch, decode_path):
    """B x ctx matrix of the reference's Qwen test (32q/8kv, D=128, P=256), scaled FP8."""

    require_gpu()
    g = torch.Generator().manual_seed(20260711 + batch)
    for ctx in (128, 256, 1024, 4096):
        per = math.ceil(ctx / 256)
        n = batch * per
        q = torch.randn(batch, 32, 128, generator=g).to(torch.bfloat16)
        k, ks = _quantize_cpu(torch.randn(n, 256, 8, 128, generator=g).to(torch.bfloat16))
        v, vs = _quantize_cpu(torch.randn(n, 256, 8, 128, generator=g).to(torch.bfloat16))
        tables = torch.randperm(n, generator=g).to(torch.int32).view(batch, per)
        lens = torch.full((batch,), ctx, dtype=torch.int32)
        got = _decode_gpu(q, k, v, ks, vs, tables, lens, 128 ** -0.5)
        assert_decode_close(got, _oracle(q, k, v, ks, vs, tables, lens, 128 ** -0.5), label=f"B{batch} ctx{ctx}")


def test_ragged_lengths_invalid_blocks_and_empty_rows(decode_path):
    """Ragged lengths (not multiples of the tile), -1 blocks inside a table, ctx=0 rows, a tiny max_context_len."""

    require_gpu()
    g = torch.Generator().manual_seed(5)
    batch, width, pool = 6, 12, 80
    q = torch.randn(batch, 32, 128, generator=g).to(torch.bfloat16)
    k, ks = _quantize_cpu(torch.randn(pool, 256, 8, 128, generator=g).to(torch.bfloat16))
    v, vs = _quantize_cpu(torch.randn(pool, 256, 8, 128, generator=g).to(torch.bfloat16))
    tables = torch.randperm(pool, generator=g)[: batch * width].to(torch.int32).view(batch, width)
    lens = torch.tensor([1, 33, 257, 3000, 0, 2900], dtype=torch.int32)
    tables[3, 2] = -1          # a hole inside a long context: skipped, not an error
    tables[5, 7:] = -1         # trailing holes
    got = _decode_gpu(q, k, v, ks, vs, tables, lens, 0.0883)
    want = _oracle(q, k, v, ks, vs, tables, lens, 0.0883)
    assert_decode_close(got, want, label="ragged")
    assert torch.all(got[4] == 0), "ctx=0 row must be zeros"
    got2 = _decode_gpu(q, k, v, ks, vs, tables, lens, 0.0883, max_ctx=40)
    assert_decode_close(got2, _oracle(q, k, v, ks, vs, tables, lens, 0.0883, max_ctx=40), label="max_ctx=40")


@pytest.mark.parametrize("qdtype", [torch.float16, torch.float32])
def test_query_dtypes_and_strided_query(qdtype, decode_path):
    require_gpu()
    g = torch.Generator().manual_seed(9)
    pool = 40
    qfull = torch.randn(3, 64, 128, generator=g).to(qdtype)
    q = qfull[:, ::2]  # non-contiguous head stride
    k, ks = _quantize_cpu(torch.randn(pool, 256, 8, 128, generator=g).to(torch.bfloat16))
    v, vs = _quantize_cpu(torch.randn(pool, 256, 8, 128, generator=g).to(torch.bfloat16))
    tables = torch.randperm(pool, generator=g)[:36].to(torch.int32).view(3, 12)
    lens = torch.tensor([700, 3072, 2048], dtype=torch.int32)
    got = _decode_gpu(q, k, v, ks, vs, tables, lens, 128 ** -0.5)
    assert got.dtype == qdtype
    assert_decode_close(got, _oracle(q, k, v, ks, vs, tables, lens, 128 ** -0.5), label=str(qdtype))


@pytest.mark.parametrize("qdtype,lo_exp,hi_exp", [(torch.bfloat16, -6.0, 4.0), (torch.float32, -3.0, 1.5)])
def test_query_magnitudes_per_head(qdtype, lo_exp, hi_exp, decode_path):
    """Query heads spanning many orders of magnitude, plus an all-zero head.

    The streaming kernel scales each query column by a power of two and splits
    it into fp8 terms for the QK MFMA (two for bf16, three for f16/f32): tiny
    heads (near-uniform softmax), huge heads (near one-hot) and a zero head
    exercise that scaling.
    """

    require_gpu()
    g = torch.Generator().manual_seed(31)
    pool, batch = 48, 4
    mags = torch.logspace(lo_exp, hi_exp, 32)
    q = torch.randn(batch, 32, 128, generator=g) * mags[None, :, None]
    q[:, 5] = 0.0
    q = q.to(qdtype)
    k, ks = _quantize_cpu(torch.randn(pool, 256, 8, 128, generator=g).to(torch.bfloat16))
    v, vs = _quantize_cpu(torch.randn(pool, 256, 8, 128, generator=g).to(torch.bfloat16))
    tables = torch.randperm(pool, generator=g)[:48].to(torch.int32).view(batch, 12)
    lens = torch.tensor([3000, 2049, 1024, 2900], dtype=torch.int32)
    got = _decode_gpu(q, k, v, ks, vs, tables, lens, 128 ** -0.5)
    assert_decode_close(got, _oracle(q, k, v, ks, vs, tables, lens, 128 ** -0.5), label=f"mags {qdtype}")


def test_small_gqa_generic_path_and_unscaled_caches():
    """head_dim 16 / page 4 (generic kernel), unit-scale FP8 and bf16 caches."""

    require_gpu()
    g = torch.Generator().manual_seed(20260625 + 16 + 4)
    q = torch.randn(3, 4, 16, generator=g).to(torch.bfloat16)
    k_src = torch.randn(9, 4, 2, 16, generator=g).to(torch.bfloat16)
    v_src = torch.randn(9, 4, 2, 16, generator=g).to(torch.bfloat16)
    tables = torch.tensor([[0, -1, -1], [1, 2, -1], [3, 4, 5]], dtype=torch.int32)
    lens = torch.tensor([1, 5, 9], dtype=torch.int32)
    # bf16 cache
    got = _decode_gpu(q, k_src, v_src, None, None, tables, lens, 0.25)
    assert_decode_close(got, _oracle(q, k_src, v_src, None, None, tables, lens, 0.25), label="bf16 cache")
    # unit-scale fp8
    k8, v8 = k_src.to(FP8), v_src.to(FP8)
    got = _decode_gpu(q, k8, v8, None, None, tables, lens, 0.25)
    assert_decode_close(got, _oracle(q, k8, v8, None, None, tables, lens, 0.25), label="unit fp8")
    # scaled fp8 at head_dim 16
    k, ks = _quantize_cpu(k_src * 9)
    v, vs = _quantize_cpu(v_src * 3)
    got = _decode_gpu(q, k, v, ks, vs, tables, lens, 0.25)
    assert_decode_close(got, _oracle(q, k, v, ks, vs, tables, lens, 0.25), label="scaled D16")


def test_unit_scale_fp8_fast_path():
    require_gpu()
    g = torch.Generator().manual_seed(21)
    q = torch.randn(2, 32, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(10, 256, 8, 128, generator=g).to(FP8)
    v = torch.randn(10, 256, 8, 128, generator=g).to(FP8)
    tables = torch.arange(10, dtype=torch.int32).view(2, 5)
    lens = torch.tensor([1111, 1280], dtype=torch.int32)
    got = _decode_gpu(q, k, v, None, None, tables, lens, 128 ** -0.5)
    assert_decode_close(got, _oracle(q, k, v, None, None, tables, lens, 128 ** -0.5), label="unit fp8 fast")


def test_unit_scale_fp8_streaming_path():
    """Unit-scale FP8 caches (no scale tensors) on the streaming kernel: ragged
    lengths, a hole, and a prefix group (virtual entries) against the oracle
    with unit scales."""

    require_gpu()
    g = torch.Generator().manual_seed(22)
    batch, width, pool = 12, 16, 200
    q = torch.randn(batch, 32, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(pool, 256, 8, 128, generator=g).to(FP8)
    v = torch.randn(pool, 256, 8, 128, generator=g).to(FP8)
    tables = torch.randperm(pool, generator=g)[: batch * width].to(torch.int32).view(batch, width).clone()
    tables[1:9:2, :3] = tables[0, :3]  # a group of 5 sharing 3 pages
    tables[10, 2] = -1
    lens = torch.randint(800, width * 256, (batch,), generator=g, dtype=torch.int32)
    lens[0] = width * 256
    set_decode_overrides(path="stream")
    got = _decode_gpu(q, k, v, None, None, tables, lens, 128 ** -0.5)
    assert_decode_close(got, _oracle(q, k, v, None, None, tables, lens, 128 ** -0.5), label="unit fp8 stream")


@pytest.mark.parametrize("name", ["decode_single", "decode_qwen_vl"])
def test_single_sequence_configs(name):
    require_gpu()
    from prism_infer import workloads

    w = getattr(workloads, name)(torch.device("cuda"))
    out = __import__("prism_infer.ops.paged_decode", fromlist=["x"]).paged_decode_attention(
        w.q, w.k_cache, w.v_cache, w.block_tables, w.context_lens, w.scale,
        k_scale_cache=w.k_scale, v_scale_cache=w.v_scale, max_context_len=w.max_context_len)
    q, k, v, ks, vs, tables, lens, mx = compact_to_cpu(w)
    assert_decode_close(out, _oracle(q, k, v, ks, vs, tables, lens, w.scale, mx), label=name)
    # the reference CPU path (bf16 dequant + SDPA in bf16) agrees within the same tolerance
    ref = oracle.decode_reference_qdtype(q, k, v, tables, lens, w.scale, k_scale_cache=ks, v_scale_cache=vs)
    assert_decode_close(out, ref, atol=3e-2, label=name + " vs bf16 reference path")


def test_mixed_batch_north_star_config(decode_path):
    """B=64, lengths U[1k,16k], 32 sequences sharing a 4096-token prefix, 8192-page pool."""

    require_gpu()
    from prism_infer.ops.paged_decode import paged_decode_attention
    from prism_infer.workloads import decode_mixed

    w = decode_mixed(torch.device("cuda"))
    out = paged_decode_attention(w.q, w.k_cache, w.v_cache, w.block_tables, w.context_lens, w.scale,
                                 k_scale_cache=w.k_scale, v_scale_cache=w.v_scale,
                                 max_context_len=w.max_context_len)
    q, k, v, ks, vs, tables, lens, mx = compact_to_cpu(w)
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens, w.scale, k_scale_cache=ks, v_scale_cache=vs,
                                          max_context_len=mx, compute_dtype=torch.float32)
    assert_decode_close(out, want, label="decode_mixed")


def test_long_context_b256_config(monkeypatch):
    """Config 5 as a chain: compaction of 64 prefixes into new dense pages, then
    decode at full shape (B=256, 32k tokens each, pages scattered in the pool)
    with sequences 0..63 starting with their compacted prefix pages.

    The compaction moved every kept slot (destination bytes equal source bytes,
    payload and scales of K and V); both kernel families agree on every
    sequence within the decode tolerance; the CPU oracle matches a sample of
    compacted and private sequences (copied pages only).
    """

    require_gpu()
    from prism_infer.ops.paged_decode import paged_decode_attention
    from prism_infer.workloads import decode_long_compacted

    w = decode_long_compacted(torch.device("cuda"))
    src, dst = w.meta["compaction_src"], w.meta["compaction_dst"]
    for cache, row in ((w.k_cache, (8, 128)), (w.v_cache, (8, 128)), (w.k_scale, (8,)), (w.v_scale, (8,))):
        flat = cache.view(torch.uint8) if cache.dtype == FP8 else cache
        flat = flat.reshape(-1, *row)
        assert torch.equal(flat.index_select(0, dst), flat.index_select(0, src)), "compacted prefix differs"
    kept = [p.physical_prompt_len for p in w.meta["compaction"].plans]
    print(f"compacted 64 prefixes: kept {sum(kept)} tokens ({min(kept)}..{max(kept)} per prefix)", flush=True)
    run = lambda: paged_decode_attention(w.q, w.k_cache, w.v_cache, w.block_tables, w.context_lens, w.scale,
                                         k_scale_cache=w.k_scale, v_scale_cache=w.v_scale,
                                         max_context_len=w.max_context_len)
    set_decode_overrides(path="stream")
    out_stream = run()
    set_decode_overrides(path="split")
    out_split = run()
    torch.cuda.synchronize()
    assert_decode_close(out_stream, out_split, label="decode_long stream vs split")
    rows = torch.tensor([0, 17, 63, 64, 255])
    pages = torch.unique(w.block_tables[rows.to(w.block_tables.device)].cpu().to(torch.int64))
    q, k, v, ks, vs, tables, lens, mx = compact_to_cpu(w, page_ids=pages)
    want = oracle.decode_kernel_semantics(q[rows], k, v, tables[rows], lens[rows], w.scale, k_scale_cache=ks,
                                          v_scale_cache=vs, max_context_len=mx, compute_dtype=torch.float32)
    assert_decode_close(out_stream[rows.to(out_stream.device)], want, label="decode_long sample (stream)")
    assert_decode_close(out_split[rows.to(out_split.device)], want, label="decode_long sample (split)")


def test_page_permutation_invariance_on_gpu():
    """Same logical K/V in different physical pages gives the same output bit for bit."""

    require_gpu()
    g = torch.Generator().manual_seed(31)
    q = torch.randn(2, 32, 128, generator=g).to(torch.bfloat16)
    k, ks = _quantize_cpu(torch.randn(16, 256, 8, 128, generator=g).to(torch.bfloat16))
    v, vs = _quantize_cpu(torch.randn(16, 256, 8, 128, generator=g).to(torch.bfloat16))
    tables = torch.arange(16, dtype=torch.int32).view(2, 8)
    lens = torch.tensor([2000, 1500], dtype=torch.int32)
    perm = torch.randperm(16, generator=g)
    inv = torch.argsort(perm)
    kp = k.view(torch.uint8)[perm].view(FP8)
    vp = v.view(torch.uint8)[perm].view(FP8)
    tables_p = inv[tables.long()].to(torch.int32)
    a = _decode_gpu(q, k, v, ks, vs, tables, lens, 0.09)
    b = _decode_gpu(q, kp, vp, ks[perm], vs[perm], tables_p, lens, 0.09)
    assert torch.equal(a, b)


def test_graph_replay_follows_device_metadata(decode_path):
    """Captured decode follows updated context_lens / max_context_len / tables on replay."""

    require_gpu()
    from prism_infer.ops.paged_decode import paged_decode_attention

    g = torch.Generator().manual_seed(20260722)
    dev = torch.device("cuda")
    q = torch.randn(2, 32, 128, generator=g).to(torch.bfloat16).to(dev)
    k, ks = _quantize_cpu(torch.randn(8, 256, 8, 128, generator=g).to(torch.bfloat16))
    v, vs = _quantize_cpu(torch.randn(8, 256, 8, 128, generator=g).to(torch.bfloat16))
    kd, vd = k.view(torch.uint8).to(dev).view(FP8), v.view(torch.uint8).to(dev).view(FP8)
    ksd, vsd = ks.to(dev), vs.to(dev)
    tables = torch.arange(8, dtype=torch.int32, device=dev).view(2, 4)
    lens = torch.tensor([4, 4], dtype=torch.int32, device=dev)
    mx = torch.tensor([4], dtype=torch.int32, device=dev)
    run = lambda: paged_decode_attention(q, kd, vd, tables, lens, 0.09, k_scale_cache=ksd, v_scale_cache=vsd,
                                         max_context_len=mx)
    run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = run()
    for new_len, swap in ((25, False), (1000, True), (700, False)):
        lens.fill_(new_len)
        mx.fill_(new_len)
        if swap:
            tables.copy_(tables.flip(0))
        graph.replay()
        torch.cuda.synchronize()
        eager = run()
        torch.cuda.synchronize()
        want = _oracle(q.cpu(), k, v, ks, vs, tables.cpu(), lens.cpu(), 0.09)
        assert_decode_close(captured, want, label=f"replay len {new_len}")
        assert torch.equal(captured.cpu(), eager.cpu())


def test_shared_prefix_groups(decode_path, monkeypatch):
    """Prefix groups in every shape the shared-page analysis must handle.

    Group A (7 members, not contiguous in the batch: virtual sequences of 4 and
    3) shares 6 pages, but one member covers only 3 whole pages, one diverges
    at page 4 and one shares only the first page; group B (3 members) shares 3
    pages; a member of B has a hole at page 1; a ctx = 0 row starts with A's
    first page; the rest are private.  Also with max_context_len cutting into
    the shared pages, and with the analysis switched off.
    """

    require_gpu()
    g = torch.Generator().manual_seed(20260811)
    pool, width, batch = 260, 12, 24
    q = torch.randn(batch, 32, 128, generator=g).to(torch.bfloat16)
    k, ks = _quantize_cpu(torch.randn(pool, 256, 8, 128, generator=g).to(torch.bfloat16))
    v, vs = _quantize_cpu(torch.randn(pool, 256, 8, 128, generator=g).to(torch.bfloat16))
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    cursor = 0

    def take(n):
        nonlocal cursor
        cursor += n
        return perm[cursor - n:cursor]

    pre_a, pre_b = take(6), take(3)
    tables = torch.full((batch, width), -1, dtype=torch.int32)
    lens = torch.zeros(batch, dtype=torch.int32)
    group_a, group_b = [0, 3, 5, 8, 11, 15, 19], [2, 9, 20]
    for b in range(batch):
        if b in group_a:
            tables[b, :6] = pre_a
            tables[b, 6:] = take(width - 6)
            lens[b] = 6 * 256 + int(torch.randint(1, 1400, (1,), generator=g))
        elif b in group_b:
            tables[b, :3] = pre_b
            tables[b, 3:] = take(width - 3)
            lens[b] = 3 * 256 + int(torch.randint(1, 2000, (1,), generator=g))
        else:
            tables[b] = take(width)
            lens[b] = int(torch.randint(1, width * 256, (1,), generator=g))
    lens[5] = 3 * 256 + 100                 # covers 3 whole shared pages
    tables[11, 4] = take(1)[0]              # diverges at page 4
    tables[13, 0] = pre_a[0]                # shares only A's first page
    lens[13] = 2000
    tables[22, 0] = pre_a[0]                # ctx = 0 row with A's first page
    lens[22] = 0
    tables[9, 1] = -1                       # B member with a hole at page 1
    assert cursor <= pool
    want = _oracle(q, k, v, ks, vs, tables, lens, 0.0883)
    got = _decode_gpu(q, k, v, ks, vs, tables, lens, 0.0883)
    assert_decode_close(got, want, label="shared groups")
    assert torch.all(got[22] == 0)
    got_cap = _decode_gpu(q, k, v, ks, vs, tables, lens, 0.0883, max_ctx=700)
    assert_decode_close(got_cap, _oracle(q, k, v, ks, vs, tables, lens, 0.0883, max_ctx=700), label="max_ctx 700")
    set_decode_overrides(path="auto", share=False)
    plain = _decode_gpu(q, k, v, ks, vs, tables, lens, 0.0883)
    assert_decode_close(plain, want, label="sharing analysis off")


def test_large_batch_prefix_groups_deterministic(monkeypatch):
    """128 sequences of ~2k-5k tokens with two prefix groups (14 members sharing
    5 pages, 21 sharing 2) on the streaming kernel: oracle parity, and
    bit-identical results across runs."""

    require_gpu()
    from prism_infer.ops.paged_decode import paged_decode_attention

    set_decode_overrides(path="stream")
    g = torch.Generator().manual_seed(20260812)
    batch, width, pool = 128, 20, 2600
    dev = torch.device("cuda")
    q = torch.randn(batch, 32, 128, generator=g).to(torch.bfloat16)
    k, ks = _quantize_cpu(torch.randn(pool, 256, 8, 128, generator=g).to(torch.bfloat16))
    v, vs = _quantize_cpu(torch.randn(pool, 256, 8, 128, generator=g).to(torch.bfloat16))
    tables = torch.randperm(pool, generator=g)[: batch * width].to(torch.int32).view(batch, width).clone()
    tables[1:40:3, :5] = tables[0, :5]       # group of 14 sharing 5 pages
    tables[70:90, :2] = tables[60, :2]       # group of 21 sharing 2 pages
    lens = torch.randint(2000, width * 256, (batch,), generator=g, dtype=torch.int32)
    to = lambda t: t.view(torch.uint8).to(dev).view(FP8) if t.dtype == FP8 else t.to(dev)
    args = (to(q), to(k), to(v), to(tables), to(lens), 0.0883)
    kw = dict(k_scale_cache=to(ks), v_scale_cache=to(vs))
    first = paged_decode_attention(*args, **kw)
    second = paged_decode_attention(*args, **kw)
    torch.cuda.synchronize()
    assert torch.equal(first, second)
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens, 0.0883, k_scale_cache=ks, v_scale_cache=vs,
                                          compute_dtype=torch.float32)
    assert_decode_close(first, want, label="large batch")


def test_plan_reuse_across_calls_and_geometries():
    """The streaming kernel's plan is kept in the per-stream workspace and reused
    while the metadata is unchanged: a call of another geometry in between (the
    per-split path, same workspace) must not disturb it, and a change of the
    metadata in place must be picked up."""

    require_gpu()
    from prism_infer.ops.paged_decode import paged_decode_attention
    from prism_infer.workloads import decode_mixed

    dev = torch.device("cuda")
    w = decode_mixed(dev)
    run = lambda: paged_decode_attention(w.q, w.k_cache, w.v_cache, w.block_tables, w.context_lens, w.scale,
                                         k_scale_cache=w.k_scale, v_scale_cache=w.v_scale,
                                         max_context_len=w.max_context_len)
    first = run()
    small = paged_decode_attention(w.q[:2], w.k_cache, w.v_cache, w.block_tables[:2], w.context_lens[:2], w.scale,
                                   k_scale_cache=w.k_scale, v_scale_cache=w.v_scale)
    again = run()
    torch.cuda.synchronize()
    assert torch.equal(first, again)
    q, k, v, ks, vs, tables, lens, mx = compact_to_cpu(w)
    want_small = oracle.decode_kernel_semantics(q[:2], k, v, tables[:2], lens[:2], w.scale, k_scale_cache=ks,
                                                v_scale_cache=vs, compute_dtype=torch.float32)
    assert_decode_close(small, want_small, label="small call in between")
    # shrink one sharing sequence below the shared prefix and another one a little
    sharing = w.meta["sharing"]
    w.context_lens[sharing[0]] = 1000
    w.context_lens[sharing[1]] -= 300
    changed = run()
    lens2 = w.context_lens.cpu()
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens2, w.scale, k_scale_cache=ks, v_scale_cache=vs,
                                          max_context_len=mx, compute_dtype=torch.float32)
    assert_decode_close(changed, want, label="metadata changed in place")
