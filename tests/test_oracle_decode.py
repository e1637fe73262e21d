"""Pins the oracle's decode formulations (oracle/kv_oracle.py) on the CPU.

Three restatements are checked against each other and against facts the
mathematics fixes, so that a dropped term, a wrong GQA index or a transposed
operand fails here:

* ``decode_kernel_semantics`` -- the reference kernel's semantics
  (prism_infer/ops/paged_decode.py:83-180) evaluated in float64;
* ``decode_reference_qdtype`` -- the reference's CPU path
  (prism_infer/ops/paged_attention_reference.py:249-320, bf16 dequant);
* ``decode_reference_fp32`` -- the reference test's oracle
  (tests/test_scaled_fp8_kv_cache.py:71-102).

Pins: explicit-loop float64 brute force on tiny shapes; ctx = 1 returns the
dequantized V row; identical keys return the mean of V; one dominant key
returns its V row; ctx = 0 and all-hole tables return zeros; page-permutation
invariance; the GQA head mapping hk = hq // G; the max_context_len bound; and
the reference's eager-vs-SDPA known-answer case (seed 20260718, atol 1e-5).
"""

from __future__ import annotations

import pytest
import torch

from oracle import (
    decode_bruteforce_f64,
    decode_kernel_semantics,
    decode_reference_fp32,
    decode_reference_qdtype,
    decode_token_mask,
    store_scaled,
)

FP8 = torch.float8_e4m3fn


def _quantized_pages(source: torch.Tensor):
    """Scaled FP8 pages of ``source`` [N, P, H, D] through the oracle store."""

    n, p, h, d = source.shape
    payload = torch.zeros(n, p, h, d, dtype=FP8)
    scales = torch.zeros(n, p, h)
    spare = torch.zeros_like(payload)
    spare_s = torch.zeros_like(scales)
    flat = source.reshape(n * p, h, d)
    store_scaled(flat, flat, payload, spare, torch.arange(n * p, dtype=torch.int32), scales, spare_s)
    return payload, scales


def _deq(payload, scales):
    """fp32 dequantization, as the kernel does it (paged_decode.py:121-139), widened to float64."""

    return (payload.float() * scales.float().unsqueeze(-1)).double()


def _case(seed, batch, hq, hkv, d, page, pool, width, lens, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, hq, d, generator=g).to(dtype)
    k, ks = _quantized_pages(torch.randn(pool, page, hkv, d, generator=g).to(dtype))
    v, vs = _quantized_pages(torch.randn(pool, page, hkv, d, generator=g).to(dtype))
    tables = torch.randperm(pool, generator=g)[: batch * width].to(torch.int32).view(batch, width)
    return q, k, v, ks, vs, tables, torch.tensor(lens, dtype=torch.int32)


def test_kernel_semantics_matches_bruteforce_small_gqa():
    """Shape of tests/test_paged_decode_kernel.py:150-161 (Hq 4, Hkv 2, D 16, P 4, ctx 1/5/9)."""

    q, k, v, ks, vs, tables, lens = _case(20260625 + 16 + 4, 3, 4, 2, 16, 4, 12, 3, [1, 5, 9])
    got = decode_kernel_semantics(q, k, v, tables, lens, 0.25, k_scale_cache=ks, v_scale_cache=vs,
                                  compute_dtype=torch.float64).double()
    kd, vd = _deq(k, ks), _deq(v, vs)
    for b in range(3):
        n = int(lens[b])
        blocks = tables[b].long()[torch.arange(n) // 4]
        keys, values = kd[blocks, torch.arange(n) % 4], vd[blocks, torch.arange(n) % 4]
        want = decode_bruteforce_f64(q[b].double(), keys, values, 0.25)
        # the kernel-semantics oracle returns q.dtype (bf16): compare at bf16 resolution
        assert torch.allclose(got[b], want, atol=2e-2, rtol=8e-3), b
    # and in float64 end to end (q promoted before the call)
    exact = decode_kernel_semantics(q.double(), k, v, tables, lens, 0.25, k_scale_cache=ks, v_scale_cache=vs)
    for b in range(3):
        n = int(lens[b])
        blocks = tables[b].long()[torch.arange(n) // 4]
        want = decode_bruteforce_f64(q[b].double(), kd[blocks, torch.arange(n) % 4], vd[blocks, torch.arange(n) % 4], 0.25)
        assert torch.allclose(exact[b], want, atol=1e-12, rtol=1e-12), b


def test_three_formulations_agree_qwen_shape():
    q, k, v, ks, vs, tables, lens = _case(20260711, 2, 32, 8, 128, 16, 20, 4, [17, 64])
    a = decode_kernel_semantics(q.double(), k, v, tables, lens, 128 ** -0.5, k_scale_cache=ks, v_scale_cache=vs)
    b = decode_reference_fp32(q, k, v, ks, vs, tables, lens, 128 ** -0.5)
    c = decode_reference_qdtype(q, k, v, tables, lens, 128 ** -0.5, k_scale_cache=ks, v_scale_cache=vs)
    assert (a - b.double()).abs().max() < 1e-2      # fp32 path, bf16 output rounding
    assert (a - c.double()).abs().max() < 3e-2      # bf16 dequant + bf16 SDPA
    assert (a - c.double()).abs().mean() < 2e-3


def test_closed_forms_ctx1_identical_keys_dominant_key():
    g = torch.Generator().manual_seed(1)
    hq, hkv, d, page = 4, 2, 8, 4
    k, ks = _quantized_pages(torch.randn(2, page, hkv, d, generator=g))
    v, vs = _quantized_pages(torch.randn(2, page, hkv, d, generator=g))
    q = torch.randn(1, hq, d, generator=g, dtype=torch.float64)
    tables = torch.tensor([[1, 0]], dtype=torch.int32)
    kd, vd = _deq(k, ks), _deq(v, vs)
    # ctx = 1: the output of every q head is the V row of its kv head (hk = hq // 2)
    out = decode_kernel_semantics(q, k, v, tables, torch.tensor([1], dtype=torch.int32), 0.3,
                                  k_scale_cache=ks, v_scale_cache=vs)
    for h in range(hq):
        assert torch.allclose(out[0, h], vd[1, 0, h // 2], atol=1e-12)
    # identical keys: uniform softmax -> mean of the attended V rows
    k_same = k.clone()
    ks_same = ks.clone()
    k_same[:] = k[0, 0]
    ks_same[:] = ks[0, 0]
    out = decode_kernel_semantics(q, k_same, v, tables, torch.tensor([6], dtype=torch.int32), 0.3,
                                  k_scale_cache=ks_same, v_scale_cache=vs)
    rows = torch.cat([vd[1], vd[0, :2]])  # logical tokens 0..5
    for h in range(hq):
        assert torch.allclose(out[0, h], rows[:, h // 2].mean(0), atol=1e-12)
    # one dominant key: a huge scale concentrates the softmax on the best-matching token
    out = decode_kernel_semantics(q, k, v, tables, torch.tensor([8], dtype=torch.int32), 1e4,
                                  k_scale_cache=ks, v_scale_cache=vs)
    keys = torch.cat([kd[1], kd[0]])
    values = torch.cat([vd[1], vd[0]])
    for h in range(hq):
        best = int(torch.argmax(keys[:, h // 2] @ q[0, h]))
        assert torch.allclose(out[0, h], values[best, h // 2], atol=1e-9)


def test_empty_rows_holes_and_bounds():
    q, k, v, ks, vs, tables, lens = _case(5, 4, 8, 2, 16, 4, 16, 4, [0, 7, 16, 9])
    tables[2] = -1                      # a row whose every block is a hole
    tables[3, 1] = -1                   # a hole inside the context: tokens 4..7 skipped
    out = decode_kernel_semantics(q.double(), k, v, tables, lens, 0.2, k_scale_cache=ks, v_scale_cache=vs)
    assert torch.all(out[0] == 0) and torch.all(out[2] == 0)
    # the hole is skipped, not an error: equals attention over tokens {0..3, 8}
    kd, vd = _deq(k, ks), _deq(v, vs)
    toks = [0, 1, 2, 3, 8]
    blocks = tables[3].long()[torch.tensor(toks) // 4]
    want = decode_bruteforce_f64(q[3].double(), kd[blocks, torch.tensor(toks) % 4], vd[blocks, torch.tensor(toks) % 4], 0.2)
    assert torch.allclose(out[3], want, atol=1e-12)
    # max_context_len bounds every row; ids >= num_blocks count as holes
    capped = decode_kernel_semantics(q.double(), k, v, tables, lens, 0.2, k_scale_cache=ks, v_scale_cache=vs,
                                     max_context_len=3)
    short = decode_kernel_semantics(q.double(), k, v, tables, torch.clamp(lens, max=3), 0.2,
                                    k_scale_cache=ks, v_scale_cache=vs)
    assert torch.equal(capped, short)
    _, valid = decode_token_mask(torch.tensor([0, 99, 1]), 12, 12, 4, 16)
    assert valid.tolist() == [True] * 4 + [False] * 4 + [True] * 4


def test_page_permutation_invariance():
    q, k, v, ks, vs, tables, lens = _case(7, 3, 8, 2, 16, 4, 12, 4, [16, 5, 11])
    perm = torch.randperm(12, generator=torch.Generator().manual_seed(8))
    inv = torch.argsort(perm)
    a = decode_kernel_semantics(q.double(), k, v, tables, lens, 0.2, k_scale_cache=ks, v_scale_cache=vs)
    b = decode_kernel_semantics(q.double(), k[perm], v[perm], inv[tables.long()].to(torch.int32), lens, 0.2,
                                k_scale_cache=ks[perm], v_scale_cache=vs[perm])
    assert torch.allclose(a, b, atol=1e-12)


def test_gqa_mapping_is_hq_div_groups():
    """Swapping two kv heads' data swaps exactly the q-head groups that read them."""

    q, k, v, ks, vs, tables, lens = _case(9, 1, 8, 2, 16, 4, 4, 3, [10])
    a = decode_kernel_semantics(q.double(), k, v, tables, lens, 0.2, k_scale_cache=ks, v_scale_cache=vs)
    sw = [1, 0]
    b = decode_kernel_semantics(q[:, [4, 5, 6, 7, 0, 1, 2, 3]].double(), k[:, :, sw], v[:, :, sw], tables, lens, 0.2,
                                k_scale_cache=ks[:, :, sw], v_scale_cache=vs[:, :, sw])
    assert torch.allclose(a[:, [4, 5, 6, 7, 0, 1, 2, 3]], b, atol=1e-12)


def test_shared_prefix_rows_equal_private_copies():
    q, k, v, ks, vs, tables, lens = _case(10, 2, 8, 2, 16, 4, 12, 3, [12, 12])
    tables[1, :2] = tables[0, :2]       # row 1 shares row 0's first two pages
    shared = decode_kernel_semantics(q.double(), k, v, tables, lens, 0.2, k_scale_cache=ks, v_scale_cache=vs)
    # private copy: duplicate those pages into fresh slots
    k2 = torch.cat([k, k[tables[0, :2].long()]])
    v2 = torch.cat([v, v[tables[0, :2].long()]])
    ks2 = torch.cat([ks, ks[tables[0, :2].long()]])
    vs2 = torch.cat([vs, vs[tables[0, :2].long()]])
    t2 = tables.clone()
    t2[1, :2] = torch.tensor([12, 13], dtype=torch.int32)
    private = decode_kernel_semantics(q.double(), k2, v2, t2, lens, 0.2, k_scale_cache=ks2, v_scale_cache=vs2)
    assert torch.allclose(shared, private, atol=1e-12)


def test_reference_eager_vs_sdpa_seed_20260718():
    """tests/test_scaled_fp8_kv_cache.py:222-280: decode after storing the current token.

    The reference attends through its eager path (a7 semantics in fp32) and
    compares with its fp32 SDPA oracle at atol/rtol 1e-5; both oracle
    formulations must meet that bound here too.
    """

    torch.manual_seed(20260718)
    q = torch.randn(1, 4, 8, dtype=torch.float32)
    current_k = torch.randn(1, 2, 8, dtype=torch.float32) * 11.0
    current_v = torch.randn_like(current_k) * 7.0
    k_source = torch.randn(2, 4, 2, 8, dtype=torch.float32) * 13.0
    v_source = torch.randn_like(k_source) * 9.0
    k, ks = _quantized_pages(k_source)
    v, vs = _quantized_pages(v_source)
    store_scaled(current_k, current_v, k, v, torch.tensor([6], dtype=torch.int32), ks, vs)
    tables = torch.tensor([[0, 1]], dtype=torch.int32)
    lens = torch.tensor([7], dtype=torch.int32)
    want = decode_reference_fp32(q, k, v, ks, vs, tables, lens, 8 ** -0.5)
    eager = decode_reference_qdtype(q, k, v, tables, lens, 8 ** -0.5, k_scale_cache=ks, v_scale_cache=vs)
    kernel = decode_kernel_semantics(q, k, v, tables, lens, 8 ** -0.5, k_scale_cache=ks, v_scale_cache=vs)
    torch.testing.assert_close(eager, want, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(kernel, want, rtol=1e-5, atol=1e-5)


def test_reference_cpu_path_rejects_what_it_rejects():
    """paged_attention_reference.py:22-63: ctx <= 0 and tables that run out raise."""

    q, k, v, ks, vs, tables, lens = _case(12, 1, 4, 2, 8, 4, 4, 2, [5])
    with pytest.raises(ValueError):
        decode_reference_qdtype(q, k, v, tables, torch.tensor([0], dtype=torch.int32), 0.3,
                                k_scale_cache=ks, v_scale_cache=vs)
    bad = tables.clone()
    bad[0, 1] = -1
    with pytest.raises(RuntimeError):
        decode_reference_qdtype(q, k, v, bad, lens, 0.3, k_scale_cache=ks, v_scale_cache=vs)
