"""GPU parity: HIP paged prefill attention against the CPU prefill oracle.

Tolerances: against the fp32-dequantisation oracle (evaluated in float64),
max |err| < 2e-2 and mean |err| < 2e-3, the bound the reference's scaled
decode test uses (tests/test_scaled_fp8_kv_cache.py, seed 20260720); against
the reference's own formulation (dequantisation in q's dtype), max |err| <
6e-2, which also covers bf16 rounding of every dequantised K/V element.
All three are multiplied by max(1, max |reference output|), so that
unit-scale caches, whose outputs reach ~8, keep the same relative bound.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

import oracle
from _helpers import require_gpu

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


def _case(seed, seqs, *, num_heads=32, num_kv_heads=8, page=256, pool=None, scaled=True, qdtype=torch.bfloat16,
          v_scale_mult=1.0, qkv_view=False):
    """Random paged history for sequences given as (query_len, context_len)."""

    g = torch.Generator().manual_seed(seed)
    pages_per = [-(-ctx // page) for _, ctx in seqs]
    width = max(pages_per)
    pool = pool or (sum(pages_per) + 7)
    perm = torch.randperm(pool, generator=g)
    tables = torch.full((len(seqs), width), -1, dtype=torch.int32)
    at = 0
    for i, n in enumerate(pages_per):
        tables[i, :n] = perm[at:at + n].to(torch.int32)
        at += n
    shape = (pool, page, num_kv_heads, 128)
    k = (torch.randn(shape, generator=g) * 2.0).to(FP8)
    v = (torch.randn(shape, generator=g) * 2.0).to(FP8)
    ks = vs = None
    if scaled:
        ks = torch.rand(shape[:-1], generator=g) * 0.2 + 0.01
        vs = (torch.rand(shape[:-1], generator=g) * 0.2 + 0.01) * v_scale_mult
    total = sum(n for n, _ in seqs)
    packed = None
    if qkv_view:
        packed = torch.randn(total, (num_heads + 2 * num_kv_heads) * 128, generator=g).to(qdtype)
        q = packed[:, :num_heads * 128].reshape(total, num_heads, 128)
    else:
        q = torch.randn(total, num_heads, 128, generator=g).to(qdtype)
    cu = torch.zeros(len(seqs) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor([n for n, _ in seqs]), 0)
    lens = torch.tensor([c for _, c in seqs], dtype=torch.int32)
    return dict(q=q, packed=packed, k=k, v=v, ks=ks, vs=vs, tables=tables, lens=lens, cu=cu,
                num_heads=num_heads, num_kv_heads=num_kv_heads)


def _run(c, scale=128 ** -0.5):
    from prism_infer.ops.paged_prefill import paged_prefill_attention

    dev = torch.device("cuda")
    ctx = SimpleNamespace(block_tables=c["tables"].to(dev), context_lens=c["lens"].to(dev),
                          cu_seqlens_q=c["cu"].to(dev))
    if c.get("packed") is not None:  # q as a strided view of the packed projection, on the device
        qd = c["packed"].to(dev)[:, :c["num_heads"] * 128].view(-1, c["num_heads"], 128)
        assert not qd.is_contiguous()
    else:
        qd = c["q"].to(dev)
    out = paged_prefill_attention(
        qd, c["k"].to(dev), c["v"].to(dev), ctx, num_heads=c["num_heads"], num_kv_heads=c["num_kv_heads"],
        scale=scale, k_scale_cache=None if c["ks"] is None else c["ks"].to(dev),
        v_scale_cache=None if c["vs"] is None else c["vs"].to(dev))
    torch.cuda.synchronize()
    return out.cpu()


def _want(c, fn, scale=128 ** -0.5):
    return fn(c["q"], c["k"], c["v"], c["tables"], c["lens"], c["cu"], num_heads=c["num_heads"],
              num_kv_heads=c["num_kv_heads"], scale=scale, k_scale_cache=c["ks"], v_scale_cache=c["vs"])


def _check(c, label, *, max_tol=2e-2, mean_tol=2e-3, ref_tol=6e-2):
    got = _run(c).float()
    want = _want(c, oracle.prefill_reference_fp32).float()
    assert got.shape == want.shape, label
    # outputs larger than 1 (unit-scale caches) carry bf16 output rounding of
    # their own size: the bounds scale with max(1, max |reference|)
    mag = max(1.0, want.abs().max().item())
    err = (got - want).abs()
    assert torch.isfinite(got).all(), f"{label}: non-finite output"
    assert err.max().item() < max_tol * mag, f"{label}: max |err| {err.max().item():.3e} (scale {mag:.2f})"
    assert err.mean().item() < mean_tol * mag, f"{label}: mean |err| {err.mean().item():.3e}"
    ref = _want(c, oracle.prefill_reference_qdtype).float()
    assert (got - ref).abs().max().item() < ref_tol * mag, f"{label}: vs q-dtype reference"


def test_prefill_mixed_lengths_gqa4():
    """Chunk after a prefix, a fresh prompt (prefix 0), a single-token chunk."""

    require_gpu()
    _check(_case(20260810, [(37, 300), (64, 64), (1, 513), (200, 1000)]), "mixed")


@pytest.mark.parametrize("heads", [(8, 8), (16, 8), (64, 8)])
def test_prefill_group_sizes(heads):
    require_gpu()
    _check(_case(20260811, [(45, 700), (33, 33)], num_heads=heads[0], num_kv_heads=heads[1]), f"heads {heads}")


@pytest.mark.parametrize("page", [16, 32, 64, 128])
def test_prefill_page_sizes(page):
    require_gpu()
    _check(_case(20260812, [(50, 77), (17, 300)], page=page), f"page {page}")


def test_prefill_unit_scale_and_f16_queries():
    require_gpu()
    _check(_case(20260813, [(40, 129), (70, 70)], scaled=False), "unit scale")
    _check(_case(20260814, [(40, 129), (70, 70)], qdtype=torch.float16), "f16 q")


@pytest.mark.parametrize("qdtype", [torch.bfloat16, torch.float16])
def test_prefill_query_magnitudes_per_head(qdtype):
    """Query heads over many orders of magnitude, an all-zero head, and a head
    whose elements spread from 2^-20 to 1 of each row's largest.

    bf16 queries reach the QK MFMA as two fp8 terms of the column scaled so
    that its largest |q| lies in [128, 256): the per-column power of two and
    the elements far below the largest (below 2^-10 of it, where the second
    term's fp8 grid no longer holds them exactly) are what these heads
    exercise; f16 queries take the 16-bit MFMA on the same data.
    """

    require_gpu()
    c = _case(20261203, [(40, 600), (70, 70)], qdtype=qdtype)
    g = torch.Generator().manual_seed(7)
    q = c["q"].float()
    tokens, heads, dim = q.shape
    q = q * torch.exp2(torch.empty(heads).uniform_(-6.0, 4.0, generator=g)).view(1, heads, 1)
    q[:, 3] = 0.0
    q[:, 5] = torch.where(q[:, 5] < 0, -1.0, 1.0) * torch.exp2(-20.0 * torch.rand(tokens, dim, generator=g)) * 4.0
    c["q"] = q.to(qdtype)
    _check(c, f"query magnitudes {qdtype}")


def test_prefill_large_v_scales_and_packed_qkv_view():
    """v scales in the thousands (P * v_scale far above f16's range, held by
    the bf16 PV operand); q is a strided view of a packed QKV projection."""

    require_gpu()
    c = _case(20260815, [(33, 200), (20, 500)], v_scale_mult=4000.0, qkv_view=True)
    got = _run(c).float()
    want = _want(c, oracle.prefill_reference_fp32).float()
    rel = (got - want).abs().max().item() / want.abs().max().item()
    assert rel < 2e-2, rel


@pytest.mark.parametrize("spread", ["mixed", "tiny"])
def test_prefill_v_scales_across_the_range(spread):
    """v scales from the 1e-6 floor to 1e4 mixed inside the same pages
    ("mixed"), or all between 1e-6 and 1e-3 ("tiny"): P * v_scale enters the
    PV MFMA as bf16, whose exponent range is fp32's, so no v scale loses
    precision to subnormals or overflows.  Checked per (token, head) relative
    to that row's largest |output| (1e-2), as the decode scale tests do."""

    require_gpu()
    c = _case(20260820 if spread == "mixed" else 20260821, [(48, 300), (17, 700), (64, 64)])
    g = torch.Generator().manual_seed(7)
    lo, hi = (-6.0, 4.0) if spread == "mixed" else (-6.0, -3.0)
    c["vs"] = torch.pow(10.0, torch.empty(c["vs"].shape).uniform_(lo, hi, generator=g))
    got = _run(c).float()
    want = _want(c, oracle.prefill_reference_fp32).float()
    assert torch.isfinite(got).all()
    row_max = want.abs().amax(dim=-1, keepdim=True)
    rel = (got - want).abs() / row_max.clamp(min=1e-30)
    print(f"[v scales {spread}] row-relative max {rel.max().item():.3e} mean {rel.mean().item():.3e}; "
          f"|out| {row_max.min().item():.3e}..{row_max.max().item():.3e}", flush=True)
    assert rel.max().item() < 1e-2 and rel.mean().item() < 1e-3


def test_prefill_long_chunk():
    """Several key tiles per query block on both sides of the diagonal."""

    require_gpu()
    _check(_case(20260816, [(700, 3000), (513, 513)]), "long")


def test_prefill_chunked_equals_full_prompt():
    """The rows of a chunk equal the same rows of a full-prompt prefill."""

    require_gpu()
    full = _case(20260817, [(600, 600)])
    chunk = dict(full)
    chunk["q"] = full["q"][400:].contiguous()
    chunk["cu"] = torch.tensor([0, 200], dtype=torch.int32)
    a = _run(full)[400:].float()
    b = _run(chunk).float()
    assert (a - b).abs().max().item() < 1e-2


def test_prefill_output_rows_follow_cu_seqlens():
    """Rows outside [cu[0], cu[B]) are not part of the result, as in the reference's concatenation."""

    require_gpu()
    c = _case(20260818, [(30, 90), (10, 40)])
    c["q"] = torch.cat([torch.randn(5, 32, 128).to(torch.bfloat16), c["q"], torch.randn(3, 32, 128).to(torch.bfloat16)])
    c["cu"] = c["cu"] + 5
    got = _run(c).float()
    want = _want(c, oracle.prefill_reference_fp32).float()
    assert got.shape == want.shape == (40, 32, 128)
    assert (got - want).abs().max().item() < 2e-2


@pytest.mark.parametrize("kind,match", [
    ("short_context", "invalid paged prefill lengths: query=30 context=20"),
    ("empty_query", "invalid paged prefill lengths: query=0 context=40"),
    ("block_past_cache", "paged KV block id exceeds cache capacity"),
    ("missing_block", "invalid block table for paged KV reference"),
])
def test_prefill_errors_match_reference(kind, match):
    require_gpu()
    c = _case(20260819, [(10, 40), (30, 300)], page=16)
    if kind == "short_context":
        c["lens"][1] = 20
    elif kind == "empty_query":
        c["cu"][1] = 0
        c["lens"][0] = 40
    elif kind == "block_past_cache":
        c["tables"][1, 3] = c["k"].shape[0] + 5
    else:
        c["tables"][1, 5] = -1
    with pytest.raises(RuntimeError, match=match):
        _run(c)
    with pytest.raises(RuntimeError, match=match.split(":")[0]):
        _want(c, oracle.prefill_reference_qdtype)


def test_prefill_chunked_workload_against_oracle_sample():
    """The bench workload (4 x (8192 prefix + 2048 chunk)); one sequence's
    last 64 query rows are checked against the oracle."""

    require_gpu()
    from prism_infer import workloads
    from prism_infer.ops.paged_prefill import paged_prefill_attention

    w = workloads.prefill_chunked(torch.device("cuda"))
    out = paged_prefill_attention(w.q, w.k_cache, w.v_cache, SimpleNamespace(
        block_tables=w.block_tables, context_lens=w.context_lens, cu_seqlens_q=w.cu_seqlens_q),
        num_heads=32, num_kv_heads=8, scale=w.scale, k_scale_cache=w.k_scale, v_scale_cache=w.v_scale)
    torch.cuda.synchronize()
    assert out.shape == w.q.shape
    seq = 2
    rows = slice(int(w.cu_seqlens_q[seq + 1]) - 64, int(w.cu_seqlens_q[seq + 1]))
    ctx = int(w.context_lens[seq])
    sub_q = w.q[rows].cpu()
    want = oracle.prefill_reference_fp32(
        sub_q, w.k_cache.cpu(), w.v_cache.cpu(), w.block_tables[seq:seq + 1].cpu(), w.context_lens[seq:seq + 1].cpu(),
        torch.tensor([0, 64], dtype=torch.int32), num_heads=32, num_kv_heads=8, scale=w.scale,
        k_scale_cache=w.k_scale.cpu(), v_scale_cache=w.v_scale.cpu())
    err = (out[rows].cpu().float() - want.float()).abs()
    assert err.max().item() < 2e-2 and err.mean().item() < 2e-3, (err.max().item(), ctx)
