"""GPU parity: seeded random paged-prefill configurations against the CPU oracles.

Each seed draws:
- kv heads 1, 2, 4 or 8 and GQA groups 1, 2, 4 or 8, which select the
  kernel's tile size and wave count;
- page sizes 16 to 256 (multiples of 16, not only powers of two), which
  select 16-, 32- or 64-key tiles;
- 1 to 5 sequences with chunk lengths 1 to 300 and prefixes 0 to 1500
  (so query blocks end mid-tile and contexts end mid-page);
- bf16 or f16 queries, scaled or unit-scale caches.

Each case is checked with the same bounds as the hand-written prefill cases
(``test_gpu_prefill._check``).
"""

from __future__ import annotations

import pytest
import torch

from _helpers import require_gpu
from test_gpu_prefill import _case, _check

pytestmark = pytest.mark.gpu


def _config(seed: int):
    g = torch.Generator().manual_seed(20261203 + seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=g))]
    hkv = pick([1, 2, 4, 8])
    groups = pick([1, 2, 4, 8])
    page = pick([16, 32, 48, 64, 96, 128, 256])
    nseq = int(torch.randint(1, 6, (1,), generator=g))
    seqs = []
    for _ in range(nseq):
        qlen = int(torch.randint(1, 301, (1,), generator=g))
        prefix = int(torch.randint(0, 1501, (1,), generator=g)) if torch.rand(1, generator=g).item() < 0.8 else 0
        seqs.append((qlen, prefix + qlen))
    qdtype = pick([torch.bfloat16, torch.bfloat16, torch.float16])
    scaled = torch.rand(1, generator=g).item() < 0.75
    return dict(seqs=seqs, num_heads=hkv * groups, num_kv_heads=hkv, page=page, qdtype=qdtype, scaled=scaled)


@pytest.mark.parametrize("seed", range(16))
def test_random_prefill_configs(seed):
    require_gpu()
    cfg = _config(seed)
    label = (f"seed {seed}: Hq={cfg['num_heads']} Hkv={cfg['num_kv_heads']} page={cfg['page']} "
             f"{cfg['qdtype']} scaled={cfg['scaled']} seqs={cfg['seqs']}")
    print(label, flush=True)
    c = _case(20261300 + seed, cfg["seqs"], num_heads=cfg["num_heads"], num_kv_heads=cfg["num_kv_heads"],
              page=cfg["page"], scaled=cfg["scaled"], qdtype=cfg["qdtype"])
    _check(c, label)


def test_many_short_sequences():
    """200 sequences (the device-side sequence lookup scans them 64 at a time),
    chunks of 1 to 40 tokens over prefixes of 0 to 300."""

    require_gpu()
    g = torch.Generator().manual_seed(20261205)
    seqs = []
    for _ in range(200):
        qlen = int(torch.randint(1, 41, (1,), generator=g))
        seqs.append((qlen, qlen + int(torch.randint(0, 301, (1,), generator=g))))
    c = _case(20261206, seqs, num_heads=16, num_kv_heads=4, page=64)
    _check(c, "200 short sequences")
