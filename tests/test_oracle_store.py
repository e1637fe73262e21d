"""Pins the oracle's scaled / unit FP8 store (oracle/kv_oracle.c) on the CPU.

Reference: ``_store_kvcache_eager`` (prism_infer/ops/kv_cache_store.py:170-230):
per (token, head) ``s = max(amax|x| / 448, 1e-6)``,
``payload = e4m3fn(clamp(x / s, -448, 448))``, slot < 0 skipped.

* the reference's own known-answer test (tests/test_scaled_fp8_kv_cache.py:149-186,
  seed 20260717) with its independent expectation (``_reference_quantize``,
  :46-61), including untouched slots keeping their prior contents;
* the unit-scale store of tests/test_fp8_kv_cache.py:31-71 (RNE cast);
* closed forms that a dropped term or swapped operand would break: the absmax
  element encodes to +-448 exactly, an all-zero row gets the 1e-6 floor and a
  zero payload, the quotient is the IEEE fp32 one (checked in float64), sign
  symmetry, and the RNE error bound |deq - x| <= 2^-4 |x| for normal payloads.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import store_scaled, store_unit

FP8 = torch.float8_e4m3fn


def _independent_quantize(tensor: torch.Tensor):
    """tests/test_scaled_fp8_kv_cache.py:46-61, written against torch's cast."""

    x = tensor.float()
    scales = torch.clamp(x.abs().amax(dim=-1) / 448.0, min=1e-6)
    payload = torch.clamp(x / scales.unsqueeze(-1), min=-448.0, max=448.0).to(FP8)
    return payload, scales


def test_reference_known_answer_seed_20260717():
    torch.manual_seed(20260717)
    key = torch.randn(5, 2, 8, dtype=torch.float32) * 37.0
    value = torch.randn_like(key) * 19.0
    cache_shape = (2, 4, 2, 8)
    k_cache = torch.full(cache_shape, -4.0, dtype=FP8)
    v_cache = torch.full(cache_shape, 4.0, dtype=FP8)
    k_scales = torch.full(cache_shape[:-1], 17.0)
    v_scales = torch.full(cache_shape[:-1], 23.0)
    slot_mapping = torch.tensor([0, 1, 4, 6, -1], dtype=torch.int32)

    store_scaled(key, value, k_cache, v_cache, slot_mapping, k_scales, v_scales)

    expected_k, expected_ks = _independent_quantize(key[:-1])
    expected_v, expected_vs = _independent_quantize(value[:-1])
    written = torch.tensor([0, 1, 4, 6])
    flat_k, flat_v = k_cache.reshape(-1, 2, 8), v_cache.reshape(-1, 2, 8)
    assert torch.equal(flat_k.index_select(0, written).view(torch.uint8), expected_k.view(torch.uint8))
    assert torch.equal(flat_v.index_select(0, written).view(torch.uint8), expected_v.view(torch.uint8))
    assert torch.equal(k_scales.reshape(-1, 2).index_select(0, written), expected_ks)
    assert torch.equal(v_scales.reshape(-1, 2).index_select(0, written), expected_vs)
    untouched = torch.tensor([2, 3, 5, 7])
    assert torch.all(flat_k.index_select(0, untouched).float() == -4.0)
    assert torch.all(flat_v.index_select(0, untouched).float() == 4.0)
    assert torch.all(k_scales.reshape(-1, 2).index_select(0, untouched) == 17.0)
    assert torch.all(v_scales.reshape(-1, 2).index_select(0, untouched) == 23.0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_store_matches_independent_quantizer_with_outliers(dtype):
    g = torch.Generator().manual_seed(20260719)
    tokens, heads, dim, pages, page = 96, 8, 128, 4, 32
    key = torch.randn(tokens, heads, dim, generator=g)
    key[torch.rand(key.shape, generator=g) < 0.01] *= 20.0
    value = torch.randn(tokens, heads, dim, generator=g) * 3.0
    key, value = key.to(dtype), value.to(dtype)
    slots = torch.randperm(pages * page, generator=g)[:tokens].to(torch.int32)
    k_cache = torch.zeros(pages, page, heads, dim, dtype=FP8)
    v_cache = torch.zeros_like(k_cache)
    ks = torch.zeros(pages, page, heads)
    vs = torch.zeros_like(ks)
    store_scaled(key, value, k_cache, v_cache, slots, ks, vs)
    ek, eks = _independent_quantize(key)
    ev, evs = _independent_quantize(value)
    idx = slots.long()
    assert torch.equal(k_cache.view(-1, heads, dim)[idx].view(torch.uint8), ek.view(torch.uint8))
    assert torch.equal(v_cache.view(-1, heads, dim)[idx].view(torch.uint8), ev.view(torch.uint8))
    assert torch.equal(ks.view(-1, heads)[idx], eks)
    assert torch.equal(vs.view(-1, heads)[idx], evs)


def test_store_closed_forms():
    g = torch.Generator().manual_seed(3)
    key = torch.randn(4, 2, 16, generator=g)
    key[1, 0] = 0.0                              # all-zero row -> floor scale, zero payload
    key[2, 1] = torch.linspace(-5.0, 3.0, 16)    # absmax is the negative end
    key[3, 0] = 1e-9                             # amax/448 below the floor
    value = -key                                 # sign symmetry
    k_cache = torch.zeros(4, 2, 16, dtype=FP8)
    v_cache = torch.zeros_like(k_cache)
    ks = torch.zeros(4, 2)
    vs = torch.zeros(4, 2)
    store_scaled(key, value, k_cache, v_cache, torch.arange(4, dtype=torch.int32), ks, vs)

    kb = k_cache.view(torch.uint8)
    # sign symmetry: V payload = K payload with the sign bit flipped (zeros: +0 vs -0)
    assert torch.equal(vs, ks)
    assert torch.equal(v_cache.float(), -k_cache.float())
    # floor
    assert ks[1, 0].item() == np.float32(1e-6)
    assert torch.all(k_cache[1, 0].float() == 0.0)
    assert ks[3, 0].item() == np.float32(1e-6)
    # the absmax element encodes to -448 exactly (0xFE), and the scale is amax / 448 in fp32
    assert kb[2, 1, 0].item() == 0xFE
    assert ks[2, 1].item() == np.float32(np.float32(5.0) / np.float32(448.0))
    # every element: payload == RNE(fp32(x / s)), where fp32(x / s) is the correctly
    # rounded quotient (a float64 quotient of fp32
    # operands rounds to the IEEE fp32 one) and within 2^-4 relative for normals
    x = key.double()
    s = ks.double().unsqueeze(-1)
    quotient = (x / s).float()
    assert torch.equal(k_cache.view(torch.uint8), quotient.clamp(-448, 448).to(FP8).view(torch.uint8))
    deq = k_cache.double() * s
    normal = quotient.abs() >= 2.0 ** -6
    assert torch.all((deq - x).abs()[normal] <= (x.abs() * 2.0 ** -4)[normal] + 1e-30)


def test_unit_scale_store_is_the_rne_cast():
    """tests/test_fp8_kv_cache.py:31-71: FP8 cache without scales stores x.to(e4m3fn)."""

    g = torch.Generator().manual_seed(20260711)
    key = (torch.randn(7, 2, 8, generator=g) * 50).to(torch.bfloat16)
    value = (torch.randn(7, 2, 8, generator=g) * 0.01).to(torch.bfloat16)
    k_cache = torch.full((3, 4, 2, 8), 2.0, dtype=FP8)
    v_cache = torch.full((3, 4, 2, 8), 2.0, dtype=FP8)
    slots = torch.tensor([11, 0, -1, 5, 6, 2, 9], dtype=torch.int32)
    store_unit(key, value, k_cache, v_cache, slots)
    keep = slots >= 0
    idx = slots[keep].long()
    assert torch.equal(k_cache.view(-1, 2, 8)[idx].view(torch.uint8), key[keep].to(FP8).view(torch.uint8))
    assert torch.equal(v_cache.view(-1, 2, 8)[idx].view(torch.uint8), value[keep].to(FP8).view(torch.uint8))
    others = torch.ones(12, dtype=torch.bool)
    others[idx] = False
    assert torch.all(k_cache.view(-1, 2, 8)[others].float() == 2.0)


def test_strided_input_and_out_of_range_slots():
    g = torch.Generator().manual_seed(11)
    packed = torch.randn(6, 3, 4, 16, generator=g).to(torch.bfloat16)  # [T, q|k|v, H, D]
    key, value = packed[:, 1], packed[:, 2]                               # token stride 192
    k_cache = torch.zeros(8, 4, 16, dtype=FP8)
    v_cache = torch.zeros_like(k_cache)
    ks = torch.full((8, 4), -1.0)
    vs = torch.full((8, 4), -1.0)
    slots = torch.tensor([7, 8, 100, -5, 0, 3], dtype=torch.int32)       # 8 and 100 are past the end
    store_scaled(key, value, k_cache, v_cache, slots, ks, vs)
    ek, eks = _independent_quantize(key)
    for t, slot in enumerate(slots.tolist()):
        if 0 <= slot < 8:
            assert torch.equal(k_cache[slot].view(torch.uint8), ek[t].view(torch.uint8))
            assert torch.equal(ks[slot], eks[t])
    written = {7, 0, 3}
    for slot in range(8):
        if slot not in written:
            assert torch.all(ks[slot] == -1.0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_torch_loop_store_equals_c_restatement(dtype):
    """The per-token torch loop (the CPU path bench.py times as the store baseline)
    writes the same bytes and scales as the C restatement, outliers, zero rows,
    skipped (-1) slots and untouched slots included."""

    from oracle import store_scaled_torch_loop

    g = torch.Generator().manual_seed(20260903)
    tokens, heads, dim, pages, page = 64, 8, 128, 3, 32
    key = torch.randn(tokens, heads, dim, generator=g)
    key[torch.rand(key.shape, generator=g) < 0.01] *= 20.0
    key[5] = 0.0
    value = torch.randn(tokens, heads, dim, generator=g) * 1e-3
    key, value = key.to(dtype), value.to(dtype)
    slots = torch.randperm(pages * page, generator=g)[:tokens].to(torch.int32)
    slots[7] = -1
    caches = []
    for fn in (store_scaled, store_scaled_torch_loop):
        kc = torch.full((pages, page, heads, dim), 0x33, dtype=torch.uint8).view(FP8)
        vc = torch.full_like(kc.view(torch.uint8), 0x44).view(FP8)
        ks = torch.full((pages, page, heads), 9.0)
        vs = torch.full_like(ks, 9.0)
        fn(key, value, kc, vc, slots, ks, vs)
        caches.append((kc.view(torch.uint8), vc.view(torch.uint8), ks, vs))
    for a, b in zip(*caches):
        assert torch.equal(a, b)
