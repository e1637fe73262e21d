"""The fp8 query split of the QK MFMAs, checked over every bf16 value (CPU).

The decode and prefill kernels multiply fp8 K rows by the query as a sum of
E4M3FN terms: each column is scaled by a power of two so that its largest
|q| lies in [128, 256), then split into terms hi, mid, ..., each the
round-to-nearest of what the previous terms left.  The products of fp8
values are exact in fp32, so the scores are exact when the terms sum to the
scaled query.  The prefill kernel uses two terms for bf16 queries and the
decode kernel three; these checks pin what each number of terms holds,
using torch's E4M3FN conversion (round to nearest even) on the whole bf16
range below 256:

- two terms hold every bf16 value of magnitude 2^-2 and up exactly (2^-10 of
  the column's largest), and are within 2^-10 below that (E4M3FN's finest
  step is the subnormal 2^-9);
- a third term never changes a bf16 value's error: the bound comes from the
  fp8 grid, not from the number of terms;
- f16 queries (11 significant bits) are not held by two terms, which is why
  the prefill kernel keeps a 16-bit MFMA for them; three terms hold them
  exactly from magnitude 2 up and within 2^-10 below.
"""

from __future__ import annotations

import torch

FP8 = torch.float8_e4m3fn


def _terms(v: torch.Tensor, n: int) -> torch.Tensor:
    """Sum of n E4M3FN terms of v, each the round-to-nearest of the remainder."""

    acc = torch.zeros_like(v)
    r = v.clone()
    for _ in range(n):
        t = r.to(FP8).float()
        acc += t
        r -= t
    return acc


def _all_below_256(dtype: torch.dtype, nbits_exp_mant: int) -> torch.Tensor:
    bits = torch.arange(0, 1 << nbits_exp_mant, dtype=torch.int32).to(torch.int16).view(dtype).float()
    bits = bits[torch.isfinite(bits) & (bits.abs() < 256)]
    return torch.cat([bits, -bits])


def test_two_terms_hold_bf16_exactly_above_the_fp8_grid():
    v = _all_below_256(torch.bfloat16, 15)
    assert v.numel() > 30000
    err2 = (v - _terms(v, 2)).abs()
    big = v.abs() >= 0.25
    assert torch.all(err2[big] == 0), "a bf16 value >= 2^-2 not held by two terms"
    assert float(err2.max()) <= 2.0 ** -10
    # the values in [128, 256) (a column's largest) and one step of bf16 below them
    top = v[(v.abs() >= 128)]
    assert torch.all(_terms(top, 2) == top)
    # one term is not enough (the split is needed at all)
    assert float((v - _terms(v, 1)).abs()[big].max()) > 0


def test_a_third_term_never_changes_a_bf16_error():
    v = _all_below_256(torch.bfloat16, 15)
    err2 = (v - _terms(v, 2)).abs()
    err3 = (v - _terms(v, 3)).abs()
    assert torch.equal(err2, err3)


def test_f16_needs_three_terms():
    v = _all_below_256(torch.float16, 15)
    big = v.abs() >= 0.25
    err2 = (v - _terms(v, 2)).abs()
    err3 = (v - _terms(v, 3)).abs()
    assert float(err2[big].max()) > 0, "two terms would hold f16 too"
    assert float(err3.max()) <= 2.0 ** -10
    # 11 significant bits in three 4-bit terms: exact while the last term's
    # step (2^-11 of the value's leading bit) stays on the fp8 grid
    assert torch.all(err3[v.abs() >= 2] == 0)
