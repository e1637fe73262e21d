"""GPU parity: the HIP KV store against the CPU oracle (bit-exact bytes and scales)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _helpers import require_gpu

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


def _run_store(key, value, cache_shape, slots, *, scaled=True, fill_k=-4.0, fill_v=4.0, fill_s=(11.0, 13.0)):
    """Run the HIP store and the oracle on the same inputs; return both results."""

    from prism_infer.ops.kv_cache_store import store_kvcache

    dev = torch.device("cuda")
    k_cache = torch.full(cache_shape, fill_k, dtype=FP8, device=dev)
    v_cache = torch.full(cache_shape, fill_v, dtype=FP8, device=dev)
    ks = torch.full(cache_shape[:-1], fill_s[0], dtype=torch.float32, device=dev)
    vs = torch.full(cache_shape[:-1], fill_s[1], dtype=torch.float32, device=dev)
    ok = k_cache.view(torch.uint8).cpu().view(FP8)
    ov = v_cache.view(torch.uint8).cpu().view(FP8)
    oks, ovs = ks.cpu(), vs.cpu()
    if scaled:
        store_kvcache(key.to(dev), value.to(dev), k_cache, v_cache, slots.to(dev), ks, vs)
        oracle.store_scaled(key.cpu(), value.cpu(), ok, ov, slots.cpu(), oks, ovs)
    else:
        store_kvcache(key.to(dev), value.to(dev), k_cache, v_cache, slots.to(dev))
        oracle.store_unit(key.cpu(), value.cpu(), ok, ov, slots.cpu())
    torch.cuda.synchronize()
    got = (k_cache.view(torch.uint8).cpu(), v_cache.view(torch.uint8).cpu(), ks.cpu(), vs.cpu())
    want = (ok.view(torch.uint8), ov.view(torch.uint8), oks, ovs)
    return got, want


def _assert_bit_exact(got, want, label):
    names = ("k payload", "v payload", "k scales", "v scales")
    for name, a, b in zip(names, got, want):
        if a.dtype == torch.float32:
            same = torch.equal(a.view(torch.int32), b.view(torch.int32))
        else:
            same = torch.equal(a, b)
        if not same:
            bad = (a.view(torch.uint8) != b.view(torch.uint8)).sum().item() if a.dtype != torch.float32 else \
                (a.view(torch.int32) != b.view(torch.int32)).sum().item()
            raise AssertionError(f"{label}: {name} differs in {bad} elements")


def test_native_fp8_encoding_matches_oracle_exhaustively():
    """Every fp32 pattern below 512 (both signs) and specials round like the oracle."""

    require_gpu()
    from prism_infer import _native

    lib = _native.lib()
    dev = torch.device("cuda")
    step = 1 << 26
    ranges = [(0, 0x44000000)]  # all non-negative fp32 < 512 (incl. subnormals, the 448..480 edge)
    for lo0, hi0 in ranges:
        for lo in range(lo0, hi0, step):
            hi = min(lo + step, hi0)
            bits = torch.arange(lo, hi, dtype=torch.int64).to(torch.int32)
            for sign in (0, -0x80000000):
                pattern = (bits | sign) if sign else bits
                vals = pattern.view(torch.float32).to(dev)
                out = torch.empty(vals.numel(), dtype=torch.uint8, device=dev)
                _native.check(lib.prism_debug_fp8_encode(vals.data_ptr(), out.data_ptr(), vals.numel(),
                                                         _native.stream_handle(dev)), "encode")
                want = oracle.e4m3fn_encode(pattern.view(torch.float32).numpy())
                got = out.cpu().numpy()
                bad = np.nonzero(got != want)[0]
                assert bad.size == 0, (
                    f"first mismatch at bits {int(pattern[bad[0]]) & 0xFFFFFFFF:#010x}: "
                    f"got {got[bad[0]]:#04x} want {want[bad[0]]:#04x} ({bad.size} total)")
    specials = np.array([np.inf, -np.inf, np.nan, -np.nan, 1e30, -1e30, 464.0, -464.0, 464.00003,
                         479.9, 480.0, 3.4e38, 0.0, -0.0, 2.0 ** -10, 2.0 ** -10 * 1.0000001], dtype=np.float32)
    specials = np.concatenate([specials, np.zeros(-len(specials) % 4, dtype=np.float32)])
    vals = torch.from_numpy(specials).to(dev)
    out = torch.empty(vals.numel(), dtype=torch.uint8, device=dev)
    _native.check(lib.prism_debug_fp8_encode(vals.data_ptr(), out.data_ptr(), vals.numel(),
                                             _native.stream_handle(dev)), "encode")
    assert np.array_equal(out.cpu().numpy(), oracle.e4m3fn_encode(specials))


def test_scaled_store_reference_case_seed_20260719():
    """The reference's Triton-store case (33 tokens, 2 heads, 16-token pages, one -1 slot)."""

    require_gpu()
    g = torch.Generator().manual_seed(20260719)
    key = (torch.randn(33, 2, 128, generator=g) * 31.0).to(torch.bfloat16)
    value = (torch.randn(33, 2, 128, generator=g) * 17.0).to(torch.bfloat16)
    slots = torch.cat([torch.arange(16), torch.arange(24, 40), torch.tensor([-1])]).to(torch.int32)
    got, want = _run_store(key, value, (3, 16, 2, 128), slots)
    _assert_bit_exact(got, want, "reference case")
    # untouched slot 20 keeps its prior contents
    assert torch.all(got[0].view(-1, 2, 128)[20].view(FP8).float() == -4.0)
    assert torch.all(got[2].view(-1, 2)[20] == 11.0)


def test_scaled_store_prefill_config_bit_exact():
    """8192 tokens with 1% outliers x20 scattered over a 512-page pool."""

    require_gpu()
    from prism_infer.workloads import store_prefill

    w = store_prefill("cpu")
    got, want = _run_store(w.key, w.value, (w.num_pages, 256, 8, 128), w.slot_mapping, fill_k=0.0, fill_v=0.0,
                           fill_s=(0.0, 0.0))
    _assert_bit_exact(got, want, "store_prefill")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_scaled_store_other_input_dtypes(dtype):
    require_gpu()
    g = torch.Generator().manual_seed(7)
    key = (torch.randn(70, 8, 128, generator=g) * 5).to(dtype)
    value = (torch.randn(70, 8, 128, generator=g) * 0.01).to(dtype)
    slots = torch.randperm(4 * 64, generator=g)[:70].to(torch.int32)
    got, want = _run_store(key, value, (4, 64, 8, 128), slots)
    _assert_bit_exact(got, want, str(dtype))


def test_scaled_store_packed_qkv_view_and_edge_rows():
    """Token stride of a packed QKV projection; zero rows, tiny rows, NaN/inf rows, -1 and out-of-range slots."""

    require_gpu()
    g = torch.Generator().manual_seed(11)
    tokens, hq, hkv, d = 24, 32, 8, 128
    qkv = torch.randn(tokens, (hq + 2 * hkv) * d, generator=g).to(torch.bfloat16)
    key = qkv[:, hq * d:(hq + hkv) * d].view(tokens, hkv, d)
    value = qkv[:, (hq + hkv) * d:].view(tokens, hkv, d)
    key[0].zero_()                      # all-zero rows -> floor scale, zero payload
    key[1, 0] = 1e-30                   # below the floor * 448
    key[2, 1, 5] = float("nan")         # NaN propagates through amax/clamp/cast
    value[3, 2, 7] = float("inf")
    value[4, 3] = -0.0
    slots = torch.arange(tokens, dtype=torch.int32) * 3
    slots[5] = -1
    slots[6] = 10_000_000  # beyond the pool: skipped
    got, want = _run_store(key, value, (2, 64, 8, 128), slots)
    _assert_bit_exact(got, want, "packed qkv")


def test_unit_scale_fp8_store_matches_cast():
    require_gpu()
    g = torch.Generator().manual_seed(20260711)
    key = (torch.randn(210, 8, 128, generator=g) * 100).to(torch.bfloat16)
    value = torch.randn(210, 8, 128, generator=g).to(torch.bfloat16)
    slots = torch.cat([torch.arange(104), torch.arange(256, 361), torch.tensor([-1])]).to(torch.int32)
    got, want = _run_store(key, value, (3, 256, 8, 128), slots, scaled=False)
    _assert_bit_exact(got[:2], want[:2], "unit fp8")


def test_dense_bf16_cache_store():
    require_gpu()
    from prism_infer.ops.kv_cache_store import store_kvcache

    g = torch.Generator().manual_seed(3)
    key = torch.randn(9, 2, 16, generator=g).to(torch.bfloat16)
    value = torch.randn(9, 2, 16, generator=g).to(torch.bfloat16)
    kc = torch.zeros(4, 4, 2, 16, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros_like(kc)
    slots = torch.tensor([0, 1, 2, 3, 8, 9, -1, 14, 15], dtype=torch.int32)
    store_kvcache(key.cuda(), value.cuda(), kc, vc, slots.cuda())
    flat_k = kc.view(-1, 2, 16).cpu()
    flat_v = vc.view(-1, 2, 16).cpu()
    for t, s in enumerate(slots.tolist()):
        if s >= 0:
            assert torch.equal(flat_k[s], key[t]) and torch.equal(flat_v[s], value[t])
    assert torch.all(flat_k[4] == 0)


def _every_bf16_below(amax: float) -> torch.Tensor:
    """All positive finite bf16 values <= amax (bf16 bit patterns 0x0001..)."""

    bits = torch.arange(1, 0x7F80, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    vals = bits[bits.float() <= amax]
    return vals


@pytest.mark.parametrize("amax", [1.0, 3.0, 448.0, 0.0625, 1.7e-5, 2.9e-38, 5.3e11, 2.0 ** 120, 2.0 ** 125,
                                  2.0 ** 126, 3.3e38])
def test_scaled_store_every_bf16_quotient(amax):
    """Each row holds ±amax and a run of bf16 values below it, so every bf16
    quotient x / s of that scale (including the ones next to fp8 rounding
    midpoints, subnormal results and scales near the fp32 range limit) goes
    through the store and must match the oracle's IEEE division bit for bit."""

    require_gpu()
    amax_bf16 = torch.tensor(amax, dtype=torch.bfloat16)
    vals = _every_bf16_below(amax_bf16.item())
    heads, dim = 8, 128
    per_row = dim - 1
    rows = -(-vals.numel() // per_row)
    rows = -(-rows // (2 * heads)) * 2 * heads  # whole tokens, K and V rows
    body = vals.repeat(-(-rows * per_row // vals.numel()))[:rows * per_row].view(rows, per_row)
    sign = torch.where(torch.arange(rows) % 3 == 0, -1.0, 1.0).to(torch.bfloat16)[:, None]
    full = torch.cat([amax_bf16.expand(rows, 1), body * sign], dim=1)
    tokens = rows // (2 * heads)
    kv = full.view(tokens, 2, heads, dim)
    key, value = kv[:, 0].contiguous(), kv[:, 1].contiguous()
    num_pages = -(-tokens // 256) + 1
    gen = torch.Generator().manual_seed(20260801)
    slots = torch.randperm(num_pages * 256, generator=gen)[:tokens].to(torch.int32)
    got, want = _run_store(key, value, (num_pages, 256, heads, dim), slots)
    _assert_bit_exact(got, want, f"every bf16 below amax={amax}")


def test_scaled_store_large_fp32_sample_bit_exact():
    """16.7M fp32 elements with per-row scales spread over 2^-30..2^30: near-
    midpoint quotients, which take the exact-division branch, occur a few
    hundred times, and every byte and scale must match the oracle."""

    require_gpu()
    gen = torch.Generator().manual_seed(20260802)
    tokens, heads, dim = 4096, 8, 128
    key = torch.randn(tokens, heads, dim, generator=gen) * torch.exp2(torch.randint(-30, 31, (tokens, heads, 1), generator=gen).float())
    value = torch.rand(tokens, heads, dim, generator=gen) * 1000.0 - 500.0
    slots = torch.randperm(20 * 256, generator=gen)[:tokens].to(torch.int32)
    got, want = _run_store(key, value, (20, 256, heads, dim), slots)
    _assert_bit_exact(got, want, "fp32 sample")
