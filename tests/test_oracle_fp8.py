"""Pins the oracle's fp32 -> E4M3FN encoder (oracle/kv_oracle.c) on the CPU.

The reference rounds with torch's own cast, ``Tensor.to(torch.float8_e4m3fn)``
(prism_infer/ops/kv_cache_store.py:222-226 and the reference test's
``_reference_quantize``, tests/test_scaled_fp8_kv_cache.py:46-61), so the
encoder is checked bit for bit against that cast: exhaustively over every
fp32 bit pattern whose magnitude lies in [2^-12, 512) -- every E4M3FN value,
every rounding midpoint and the overflow edge 448 < x <= 464 < x lie there --
and on a strided sample of the rest (tiny values, large values, inf, NaN).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import e4m3fn_decode_table, e4m3fn_encode, e4m3fn_encode_bit_range

CHUNK = 1 << 25


def _torch_bits(lo: int, hi: int) -> np.ndarray:
    x = torch.from_numpy(np.arange(lo, hi, dtype=np.uint64).astype(np.uint32).view(np.float32))
    return x.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _check_range(lo: int, hi: int) -> None:
    for start in range(lo, hi, CHUNK):
        end = min(hi, start + CHUNK)
        got = e4m3fn_encode_bit_range(start, end)
        want = _torch_bits(start, end)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, (
            f"bits 0x{start + int(bad[0]):08x}: oracle 0x{got[bad[0]]:02x} torch 0x{want[bad[0]]:02x}"
        )


@pytest.mark.parametrize("sign", [0, 1], ids=["positive", "negative"])
def test_encoder_exhaustive_over_the_fp8_range(sign):
    lo = (127 - 12) << 23  # 2^-12
    hi = (127 + 9) << 23   # 512
    base = sign << 31
    _check_range(base | lo, base | hi)


def test_encoder_sampled_outside_the_fp8_range():
    rng = np.random.default_rng(20260717)
    pieces = [
        np.arange(0, (127 - 12) << 23, 4099, dtype=np.uint64),             # tiny and subnormal fp32
        np.arange((127 + 9) << 23, 0x7F800000, 4099, dtype=np.uint64),     # >= 512
        np.array([0x7F800000, 0x7F800001, 0x7FC00000, 0x7FFFFFFF], dtype=np.uint64),  # inf, NaNs
        rng.integers(0, 1 << 31, 1 << 20, dtype=np.uint64),
    ]
    bits = np.concatenate(pieces).astype(np.uint32)
    bits = np.concatenate([bits, bits | np.uint32(0x80000000)])
    values = bits.view(np.float32)
    got = e4m3fn_encode(values)
    want = torch.from_numpy(values.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, f"bits 0x{bits[bad[0]]:08x}: oracle 0x{got[bad[0]]:02x} torch 0x{want[bad[0]]:02x}"


def test_decode_table_matches_torch_and_the_format():
    table = e4m3fn_decode_table()
    want = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(table), np.isnan(want))
    finite = ~np.isnan(want)
    assert np.array_equal(table[finite], want[finite])
    # format facts: 0x7E = 448 (largest finite), 0x01 = 2^-9 (smallest subnormal),
    # 0x08 = 2^-6 (smallest normal), 0x7F/0xFF are the only NaN codes
    assert table[0x7E] == 448.0 and table[0xFE] == -448.0
    assert table[0x01] == 2.0 ** -9 and table[0x08] == 2.0 ** -6
    assert np.flatnonzero(np.isnan(table)).tolist() == [0x7F, 0xFF]


def test_round_trip_of_every_code():
    table = e4m3fn_decode_table()
    codes = np.arange(256, dtype=np.uint8)
    finite = ~np.isnan(table)
    again = e4m3fn_encode(table[finite])
    # +0 and -0 keep their sign bit; every finite code maps back to itself
    assert np.array_equal(again, codes[finite])


def test_ties_round_to_even_and_overflow_edge():
    cases = {
        1.0 + 1.0 / 16: 0x38,    # midpoint of 1.0 (even) and 1.125 -> 1.0
        1.0 + 3.0 / 16: 0x3A,    # midpoint of 1.125 and 1.25 (even) -> 1.25
        2.0 ** -10: 0x00,        # half the smallest subnormal -> +0 (even)
        3 * 2.0 ** -10: 0x02,    # midpoint of 2^-9 and 2^-8 (even) -> 2^-8
        448.0: 0x7E,
        464.0: 0x7E,             # midpoint of 448 and the NaN slot: ties to 448
        464.0001: 0x7F,          # above the midpoint: NaN (no saturation in the cast)
        float("inf"): 0x7F,
    }
    values = np.array(list(cases), dtype=np.float32)
    got = e4m3fn_encode(values)
    assert got.tolist() == list(cases.values())
    assert e4m3fn_encode(-values).tolist() == [c | 0x80 for c in cases.values()]
