"""GPU parity of one layer's decode step (store the step's K/V, then paged
decode), eagerly and captured in a graph that is replayed with refilled
metadata, padded rows included.

Expectations come from the CPU oracle (oracle.store_scaled then
oracle.decode_kernel_semantics); the first case restates the reference's
decode-after-store test (tests/test_scaled_fp8_kv_cache.py:222-280,
seed 20260718, atol/rtol 1e-5).
"""

from __future__ import annotations

import pytest
import torch

from prism_infer.ops.paged_decode import set_decode_overrides

import oracle
from _helpers import assert_decode_close, require_gpu

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


def _dev(t):
    return t.view(torch.uint8).cuda().view(FP8) if t.dtype == FP8 else t.cuda()


def _quantize(source):
    n, p, h, d = source.shape
    k = torch.zeros(n, p, h, d, dtype=FP8)
    s = torch.zeros(n, p, h)
    flat = source.reshape(n * p, h, d)
    oracle.store_scaled(flat, flat, k, torch.zeros_like(k), torch.arange(n * p, dtype=torch.int32), s,
                        torch.zeros_like(s))
    return k, s


def test_reference_decode_after_store_seed_20260718():
    require_gpu()
    from prism_infer.engine.decode_attention import PagedKVDecodeAttention, pack_decode_metadata

    torch.manual_seed(20260718)
    q = torch.randn(1, 4, 8, dtype=torch.float32)
    current_k = torch.randn(1, 2, 8, dtype=torch.float32) * 11.0
    current_v = torch.randn_like(current_k) * 7.0
    k_source = torch.randn(2, 4, 2, 8, dtype=torch.float32) * 13.0
    v_source = torch.randn_like(k_source) * 9.0
    k, ks = _quantize(k_source)
    v, vs = _quantize(v_source)
    layer = PagedKVDecodeAttention(num_heads=4, num_kv_heads=2, head_dim=8, scale=8 ** -0.5)
    layer.k_cache, layer.v_cache = _dev(k), _dev(v)
    layer.k_scale_cache, layer.v_scale_cache = _dev(ks), _dev(vs)
    meta = pack_decode_metadata([6], [7], [[0, 1]], device="cuda")
    got = layer(q.cuda(), current_k.cuda(), current_v.cuda(), meta)
    torch.cuda.synchronize()
    # expected: the oracle's store of the current token, then the reference test's fp32 oracle
    ek, ev, eks, evs = k.clone(), v.clone(), ks.clone(), vs.clone()
    oracle.store_scaled(current_k, current_v, ek, ev, torch.tensor([6], dtype=torch.int32), eks, evs)
    assert torch.equal(layer.k_cache.view(torch.uint8).cpu(), ek.view(torch.uint8))
    assert torch.equal(layer.v_scale_cache.cpu(), evs)
    want = oracle.decode_reference_fp32(q, ek, ev, eks, evs, torch.tensor([[0, 1]], dtype=torch.int32),
                                        torch.tensor([7], dtype=torch.int32), 8 ** -0.5)
    torch.testing.assert_close(got.cpu(), want, rtol=1e-5, atol=1e-5)


def _step_case(g, batch, width, pool, active):
    """Random metadata for a padded batch: rows >= active get slot -1 and ctx 0."""

    perm = torch.randperm(pool, generator=g)
    tables, slots, lens = [], [], []
    cursor = 0
    for b in range(batch):
        if b >= active:
            tables.append([])
            slots.append(-1)
            lens.append(0)
            continue
        n = int(torch.randint(1, width * 256, (1,), generator=g))
        pages = (n + 255) // 256
        row = perm[cursor:cursor + pages].tolist()
        cursor += pages
        tables.append(row)
        lens.append(n)
        slots.append(row[(n - 1) // 256] * 256 + (n - 1) % 256)  # the step's token is the last one
    return slots, lens, tables


@pytest.mark.parametrize("path", ["auto", "stream"])
def test_graph_captured_store_and_decode_replays(path, monkeypatch):
    """A layer's store + decode captured once at batch 8, replayed for three
    steps with different metadata and K/V, padded rows included."""

    require_gpu()
    from prism_infer.engine.decode_attention import PagedKVDecodeAttention, pack_decode_metadata

    if path == "stream":
        set_decode_overrides(path="stream")
    g = torch.Generator().manual_seed(20260813)
    batch, width, pool = 8, 6, 64
    k_src = torch.randn(pool, 256, 8, 128, generator=g).to(torch.bfloat16)
    v_src = torch.randn(pool, 256, 8, 128, generator=g).to(torch.bfloat16)
    k, ks = _quantize(k_src)
    v, vs = _quantize(v_src)
    layer = PagedKVDecodeAttention(32, 8, 128, 128 ** -0.5)
    layer.k_cache, layer.v_cache = _dev(k), _dev(v)
    layer.k_scale_cache, layer.v_scale_cache = _dev(ks), _dev(vs)
    q = torch.zeros(batch, 32, 128, dtype=torch.bfloat16, device="cuda")
    kk = torch.zeros(batch, 8, 128, dtype=torch.bfloat16, device="cuda")
    vv = torch.zeros_like(kk)
    meta = pack_decode_metadata(*_step_case(g, batch, width, pool, batch), width=width, device="cuda")
    layer(q, kk, vv, meta)  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = layer(q, kk, vv, meta)
    cpu_k, cpu_v, cpu_ks, cpu_vs = (layer.k_cache.view(torch.uint8).cpu().view(FP8), layer.v_cache.view(torch.uint8).cpu().view(FP8),
                                    layer.k_scale_cache.cpu(), layer.v_scale_cache.cpu())
    for step, active in enumerate((8, 5, 2)):
        slots, lens, tables = _step_case(g, batch, width, pool, active)
        step_q = torch.randn(batch, 32, 128, generator=g).to(torch.bfloat16)
        step_k = torch.randn(batch, 8, 128, generator=g).to(torch.bfloat16)
        step_v = torch.randn(batch, 8, 128, generator=g).to(torch.bfloat16)
        q.copy_(step_q)
        kk.copy_(step_k)
        vv.copy_(step_v)
        meta.copy_(pack_decode_metadata(slots, lens, tables, width=width, device="cuda"))
        graph.replay()
        torch.cuda.synchronize()
        # oracle: the same store, then decode over the updated pages
        oracle.store_scaled(step_k, step_v, cpu_k, cpu_v, torch.tensor(slots, dtype=torch.int32), cpu_ks, cpu_vs)
        assert torch.equal(layer.k_cache.view(torch.uint8).cpu(), cpu_k.view(torch.uint8)), f"step {step}: K pages"
        assert torch.equal(layer.v_scale_cache.cpu(), cpu_vs), f"step {step}: V scales"
        t = pack_decode_metadata(slots, lens, tables, width=width)
        want = oracle.decode_kernel_semantics(step_q, cpu_k, cpu_v, t.block_tables, t.context_lens, 128 ** -0.5,
                                              k_scale_cache=cpu_ks, v_scale_cache=cpu_vs,
                                              max_context_len=int(t.max_context_len), compute_dtype=torch.float32)
        assert_decode_close(out, want, label=f"replay {step} ({active} active rows)")
        assert torch.all(out[active:] == 0), "padded rows must be zeros"
