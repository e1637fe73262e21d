"""GPU parity of paged decode across the whole range of K and V scales.

The streaming kernel multiplies P * v_scale into its PV MFMA as one 16-bit
value.  An f16 operand would overflow for v scales above 255 (|V| > 1.1e5,
P <= 2^8 with the lazy softmax rescaling) and lose precision towards f16
subnormals for v scales far below 1; a tile-wide power-of-two shift cannot
fix both at once when a tile mixes a huge-V token of low weight with a
tiny-V token of high weight.  The kernel therefore uses bf16 (fp32's exponent
range).  These cases mix, inside the same tiles and pages, rows with v scales
in [255, 1e4], rows near the largest scale (|V| ~ 4.5e6), rows at the 1e-6
scale floor and rows of zeros, plus whole pages of huge and of tiny rows, and
K scales up to 1e4, so that the dominant token of a row is sometimes a tiny-V
one next to huge-V neighbours.  Every kernel family is compared with the
float64 oracle of the kernel semantics (prism_infer/ops/paged_decode.py:83-180)
per (sequence, head) relative to that row's largest |output|: the decode
tolerance (tests/test_scaled_fp8_kv_cache.py:470-472: 1e-2 relative) scaled to
the row, so that tiny rows are held to the same relative accuracy as unit
rows and huge rows are not failed by an absolute bound.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from _helpers import require_gpu
from prism_infer.ops.paged_decode import set_decode_overrides

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn
PAGE = 256


def _quantize(source: torch.Tensor):
    n, p, h, d = source.shape
    flat = source.reshape(n * p, h, d)
    q8 = torch.zeros(n, p, h, d, dtype=FP8)
    s = torch.zeros(n, p, h, dtype=torch.float32)
    q8b = torch.zeros_like(q8)
    sb = torch.zeros_like(s)
    oracle.store_scaled(flat, flat, q8, q8b, torch.arange(n * p, dtype=torch.int32), s, sb)
    return q8, s


def _row_factors(g: torch.Generator, n: int, heads: int, kind: str) -> torch.Tensor:
    """Per (token, head) magnitude factors for N(0,1) rows (amax of 128 N(0,1) ~ 3)."""

    u = torch.rand(n, heads, generator=g)
    f = torch.ones(n, heads)
    if kind == "v":
        # v scale = amax / 448: [255, 1e4] <-> factor ~ [3.8e4, 1.5e6]
        big = torch.exp(torch.empty(n, heads).uniform_(torch.log(torch.tensor(3.8e4)).item(),
                                                       torch.log(torch.tensor(1.5e6)).item(), generator=g))
        tiny = torch.exp(torch.empty(n, heads).uniform_(torch.log(torch.tensor(1e-7)).item(),
                                                        torch.log(torch.tensor(1e-2)).item(), generator=g))
        f = torch.where(u < 0.2, big, f)
        f = torch.where((u >= 0.2) & (u < 0.25), torch.full_like(f, 1.45e6), f)  # near the 1e4 scale
        f = torch.where((u >= 0.25) & (u < 0.45), tiny, f)
        f = torch.where((u >= 0.45) & (u < 0.5), torch.zeros_like(f), f)       # floor-scaled zero rows
    else:
        # k scales up to 1e4
        big = torch.exp(torch.empty(n, heads).uniform_(0.0, torch.log(torch.tensor(1.5e6)).item(), generator=g))
        f = torch.where(u < 0.2, big, f)
    return f


def _case(seed: int):
    g = torch.Generator().manual_seed(seed)
    batch, hq, hkv, d, width = 8, 32, 8, 128, 16
    pool = batch * width + 4
    q = torch.randn(batch, hq, d, generator=g).to(torch.bfloat16)
    n_tok = pool * PAGE
    kf = _row_factors(g, n_tok, hkv, "k").view(pool, PAGE, hkv, 1)
    vf = _row_factors(g, n_tok, hkv, "v").view(pool, PAGE, hkv, 1)
    # whole pages whose every v scale is out of range: huge, tiny, floor
    vf[3] = 1.2e6
    vf[5] = 1e-4
    vf[7] = 1e-8
    k_src = (torch.randn(pool, PAGE, hkv, d, generator=g) * kf).to(torch.bfloat16)
    v_src = (torch.randn(pool, PAGE, hkv, d, generator=g) * vf).to(torch.bfloat16)
    k, ks = _quantize(k_src)
    v, vs = _quantize(v_src)
    assert 255.0 < float(vs.max()) < 3e4 and float(vs.min()) == pytest.approx(1e-6)
    assert float(ks.max()) > 1e3
    tables = torch.randperm(pool, generator=g)[: batch * width].to(torch.int32).view(batch, width)
    # every sequence reads the special pages somewhere
    for b in range(batch):
        tables[b, b % width] = (3, 5, 7)[b % 3]
    lens = torch.randint(PAGE, width * PAGE + 1, (batch,), generator=g).to(torch.int32)
    lens[0] = width * PAGE
    return q, k, v, ks, vs, tables, lens


def _run(q, k, v, ks, vs, tables, lens, scale):
    from prism_infer.ops.paged_decode import paged_decode_attention

    dev = torch.device("cuda")
    to = lambda t: t.view(torch.uint8).to(dev).view(FP8) if t.dtype == FP8 else t.to(dev)
    out = paged_decode_attention(to(q), to(k), to(v), to(tables), to(lens), scale, k_scale_cache=to(ks),
                                 v_scale_cache=to(vs))
    torch.cuda.synchronize()
    return out.cpu().float()


def _assert_row_relative(got: torch.Tensor, want: torch.Tensor, label: str, rtol: float = 1e-2) -> None:
    assert torch.isfinite(got).all(), f"{label}: non-finite output"
    want = want.float()
    row_max = want.abs().amax(dim=-1, keepdim=True)
    err = (got - want).abs()
    zero_rows = row_max == 0
    assert torch.all(err[zero_rows.expand_as(err)] == 0), f"{label}: nonzero output for an all-zero row"
    rel = (err / row_max.clamp(min=1e-38)).masked_fill(zero_rows, 0.0)
    worst = float(rel.max())
    mean = float(rel.mean())
    print(f"[{label}] row-relative max {worst:.3e} mean {mean:.3e}; |out| from "
          f"{float(row_max[~zero_rows].min()):.3e} to {float(row_max.max()):.3e}", flush=True)
    assert worst <= rtol, f"{label}: row-relative error {worst:.3e} > {rtol}"
    assert mean <= rtol / 10, f"{label}: mean row-relative error {mean:.3e}"


@pytest.mark.parametrize("path", ["auto", "stream", "split"])
def test_extreme_k_and_v_scales_all_families(path):
    require_gpu()
    q, k, v, ks, vs, tables, lens = _case(20260901)
    scale = 128 ** -0.5
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens, scale, k_scale_cache=ks, v_scale_cache=vs)
    set_decode_overrides(path=path)
    got = _run(q, k, v, ks, vs, tables, lens, scale)
    _assert_row_relative(got, want, f"extreme scales path={path}")


def test_extreme_scales_generic_family():
    """The generic kernel (no split-K, fp32 PV) on the same pages with a GQA group it alone serves (G = 32)."""

    require_gpu()
    q, k, v, ks, vs, tables, lens = _case(20260902)
    # 32 query heads over 1 kv head: G = 32 > 16 leaves the fast families
    k1, v1 = k[:, :, :1].contiguous(), v[:, :, :1].contiguous()
    ks1, vs1 = ks[:, :, :1].contiguous(), vs[:, :, :1].contiguous()
    scale = 128 ** -0.5
    want = oracle.decode_kernel_semantics(q, k1, v1, tables, lens, scale, k_scale_cache=ks1, v_scale_cache=vs1)
    got = _run(q, k1, v1, ks1, vs1, tables, lens, scale)
    _assert_row_relative(got, want, "extreme scales generic")
