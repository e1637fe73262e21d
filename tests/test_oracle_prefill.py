"""Pins for the paged-prefill oracle (CPU only).

Each check would catch a plausible slip in the restatement of
paged_prefill_attention_reference (ops/paged_attention_reference.py:185-246):
an off-by-one in the causal bound, a wrong prefix, a head mapping error, a
transposed operand or a mis-gathered page.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import oracle

FP8 = torch.float8_e4m3fn


def _case(seed, seqs, *, num_heads=4, num_kv_heads=2, page=16, dim=16, scaled=True):
    g = torch.Generator().manual_seed(seed)
    pages_per = [-(-ctx // page) for _, ctx in seqs]
    pool = sum(pages_per) + 3
    perm = torch.randperm(pool, generator=g)
    tables = torch.full((len(seqs), max(pages_per)), -1, dtype=torch.int32)
    at = 0
    for i, n in enumerate(pages_per):
        tables[i, :n] = perm[at:at + n].to(torch.int32)
        at += n
    shape = (pool, page, num_kv_heads, dim)
    k = torch.randn(shape, generator=g).to(FP8)
    v = torch.randn(shape, generator=g).to(FP8)
    ks = torch.rand(shape[:-1], generator=g) + 0.5 if scaled else None
    vs = torch.rand(shape[:-1], generator=g) + 0.5 if scaled else None
    q = torch.randn(sum(n for n, _ in seqs), num_heads, dim, generator=g)
    cu = torch.zeros(len(seqs) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor([n for n, _ in seqs]), 0)
    lens = torch.tensor([c for _, c in seqs], dtype=torch.int32)
    return dict(q=q, k=k, v=v, ks=ks, vs=vs, tables=tables, lens=lens, cu=cu, nh=num_heads, nkv=num_kv_heads)


def _run(c, fn, scale=0.3, q=None):
    return fn(c["q"] if q is None else q, c["k"], c["v"], c["tables"], c["lens"], c["cu"], num_heads=c["nh"],
              num_kv_heads=c["nkv"], scale=scale, k_scale_cache=c["ks"], v_scale_cache=c["vs"])


def _dense(c, i):
    """Sequence i's dequantised history, gathered by hand (fp32)."""

    page = c["k"].shape[1]
    ctx = int(c["lens"][i])
    rows = [(int(c["tables"][i, t // page]), t % page) for t in range(ctx)]
    keys = torch.stack([c["k"][b, r].float() * (c["ks"][b, r].unsqueeze(-1) if c["ks"] is not None else 1) for b, r in rows])
    values = torch.stack([c["v"][b, r].float() * (c["vs"][b, r].unsqueeze(-1) if c["vs"] is not None else 1) for b, r in rows])
    return keys, values


def test_prefill_matches_bruteforce_f64():
    c = _case(1, [(3, 7), (4, 4), (1, 18)], dim=8)
    got = _run(c, oracle.prefill_reference_fp32).double()
    for i in range(3):
        keys, values = _dense(c, i)
        s, e = int(c["cu"][i]), int(c["cu"][i + 1])
        want = oracle.prefill_bruteforce_f64(c["q"][s:e].double(), keys.double(), values.double(),
                                             int(c["lens"][i]) - (e - s), 0.3)
        assert torch.allclose(got[s:e], want, atol=1e-6), i


def test_single_query_chunk_is_decode():
    """A one-token chunk at the end of the history is a decode step."""

    c = _case(2, [(1, 40), (1, 17), (1, 16)])
    got = _run(c, oracle.prefill_reference_fp32)
    want = oracle.decode_kernel_semantics(c["q"], c["k"], c["v"], c["tables"], c["lens"], 0.3,
                                          k_scale_cache=c["ks"], v_scale_cache=c["vs"])
    assert torch.allclose(got, want, atol=1e-6)
    got_q = _run(c, oracle.prefill_reference_qdtype)
    want_q = oracle.decode_reference_qdtype(c["q"], c["k"], c["v"], c["tables"], c["lens"], 0.3,
                                            k_scale_cache=c["ks"], v_scale_cache=c["vs"])
    assert torch.allclose(got_q, want_q, atol=1e-5)


def test_fresh_prompt_is_causal_sdpa():
    """Prefix 0: the library's causal SDPA over the gathered history."""

    c = _case(3, [(20, 20), (9, 9)])
    got = _run(c, oracle.prefill_reference_fp32).float()
    for i in range(2):
        keys, values = _dense(c, i)
        s, e = int(c["cu"][i]), int(c["cu"][i + 1])
        g = c["nh"] // c["nkv"]
        want = F.scaled_dot_product_attention(
            c["q"][s:e].transpose(0, 1).unsqueeze(0), keys.repeat_interleave(g, 1).transpose(0, 1).unsqueeze(0),
            values.repeat_interleave(g, 1).transpose(0, 1).unsqueeze(0), is_causal=True, scale=0.3)
        assert torch.allclose(got[s:e], want.squeeze(0).transpose(0, 1), atol=1e-5), i


def test_chunk_equals_rows_of_full_prompt():
    c = _case(4, [(50, 50)])
    full = _run(c, oracle.prefill_reference_fp32)
    chunk = dict(c)
    chunk["cu"] = torch.tensor([0, 18], dtype=torch.int32)
    part = _run(chunk, oracle.prefill_reference_fp32, q=c["q"][32:])
    assert torch.allclose(full[32:], part, atol=1e-6)


def test_page_permutation_invariance():
    c = _case(5, [(6, 40), (5, 21)])
    base = _run(c, oracle.prefill_reference_fp32)
    perm = torch.randperm(c["k"].shape[0], generator=torch.Generator().manual_seed(9))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    moved = dict(c)
    for name in ("k", "v", "ks", "vs"):
        moved[name] = c[name][perm]
    moved["tables"] = torch.where(c["tables"] >= 0, inv[c["tables"].clamp(min=0).long()].to(torch.int32), c["tables"])
    assert torch.equal(base, _run(moved, oracle.prefill_reference_fp32))


def test_gqa_head_mapping():
    """Query head h reads kv head h // G: zeroing kv head 1's values changes
    exactly the outputs of query heads G..2G-1."""

    c = _case(6, [(5, 30)], num_heads=6, num_kv_heads=3)
    base = _run(c, oracle.prefill_reference_fp32)
    c2 = dict(c)
    c2["v"] = c["v"].clone()
    c2["v"][:, :, 1] = torch.zeros((), dtype=FP8)
    out = _run(c2, oracle.prefill_reference_fp32)
    changed = (out - base).abs().amax(dim=(0, 2)) > 0
    assert changed.tolist() == [False, False, True, True, False, False]


def test_qdtype_formulation_within_bf16_rounding():
    c = _case(7, [(12, 50)], dim=32)
    c["q"] = c["q"].to(torch.bfloat16)
    a = _run(c, oracle.prefill_reference_fp32).float()
    b = _run(c, oracle.prefill_reference_qdtype).float()
    assert (a - b).abs().max().item() < 3e-2


@pytest.mark.parametrize("kind,match", [
    ("short_context", "invalid paged prefill lengths: query=6 context=4"),
    ("empty_query", "invalid paged prefill lengths: query=0"),
    ("block_past_cache", "paged KV block id exceeds cache capacity"),
    ("missing_block", "invalid block table for paged KV reference"),
])
def test_reference_errors(kind, match):
    c = _case(8, [(3, 20), (6, 40)])
    if kind == "short_context":
        c["lens"][1] = 4
    elif kind == "empty_query":
        c["cu"][1] = 0
    elif kind == "block_past_cache":
        c["tables"][1, 1] = c["k"].shape[0]
    else:
        c["tables"][1, 1] = -1
    for fn in (oracle.prefill_reference_fp32, oracle.prefill_reference_qdtype):
        with pytest.raises(RuntimeError, match=match):
            _run(c, fn)
