"""GPU parity of the split-K kernel's in-kernel chunk merge.

The split-K kernel runs one workgroup per (sequence, kv head, chunk of
tokens); when a sequence has more than one live chunk, each chunk writes an
(m, l, acc) partial and the last chunk to arrive on the (sequence, kv head)
counter merges them.  These cases drive that merge:

- many chunks per sequence (a 256-token split over contexts up to 40k tokens:
  up to 157 live chunks, so the merge takes several rounds of loads in every
  chunk group), for GQA groups 1, 3, 4 and 16;
- ragged lengths whose last chunk is short or holds a single token, empty
  sequences and holes (-1 block ids) that leave whole chunks without an
  attended token (m = -inf partials);
- a workspace full of arbitrary bytes, including bytes left behind by the
  streaming kernel on the same workspace: the counters carry a per-call tag,
  so no clearing is needed, and the result is bit-identical to a call on a
  fresh zeroed workspace.

Each output is checked against ``decode_kernel_semantics`` (the float64
oracle of prism_infer/ops/paged_decode.py:83-180) within the decode tolerance
of tests/test_scaled_fp8_kv_cache.py:470-472.
"""

from __future__ import annotations

import math

import pytest
import torch

import oracle
from _helpers import assert_decode_close, require_gpu
from prism_infer.ops.paged_decode import set_decode_overrides

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


def _quantize(src: torch.Tensor):
    n, p, h, d = src.shape
    flat = src.reshape(n * p, h, d)
    q8 = torch.zeros(n, p, h, d, dtype=FP8)
    s = torch.zeros(n, p, h, dtype=torch.float32)
    q8b, sb = torch.zeros_like(q8), torch.zeros_like(s)
    oracle.store_scaled(flat, flat, q8, q8b, torch.arange(n * p, dtype=torch.int32), s, sb)
    return q8, s


def _case(seed: int, batch: int, hkv: int, groups: int, max_len: int, page: int = 256, holes: float = 0.0):
    g = torch.Generator().manual_seed(seed)
    width = math.ceil(max_len / page)
    pool = batch * width + 2
    q = torch.randn(batch, hkv * groups, 128, generator=g).to(torch.bfloat16)
    k, ks = _quantize(torch.randn(pool, page, hkv, 128, generator=g).to(torch.bfloat16))
    v, vs = _quantize(torch.randn(pool, page, hkv, 128, generator=g).to(torch.bfloat16))
    tables = torch.randperm(pool, generator=g)[: batch * width].to(torch.int32).view(batch, width).clone()
    if holes:
        tables[torch.rand(batch, width, generator=g) < holes] = -1
    lens = torch.randint(1, max_len + 1, (batch,), generator=g, dtype=torch.int32)
    lens[0] = max_len
    return q, k, v, ks, vs, tables, lens


def _to_gpu(*ts):
    dev = torch.device("cuda")
    return [t.view(torch.uint8).to(dev).view(FP8) if t.dtype == FP8 else t.to(dev) for t in ts]


def _run(q, k, v, ks, vs, tables, lens, scale, workspace=None):
    from prism_infer.ops.paged_decode import _launch_paged_decode_attention

    qd, kd, vd, ksd, vsd, td, ld = _to_gpu(q, k, v, ks, vs, tables, lens)
    mx = torch.tensor([tables.shape[1] * k.shape[1]], dtype=torch.int32, device=qd.device)
    out = _launch_paged_decode_attention(qd, kd, vd, td, ld, scale, mx, k_scale_cache=ksd, v_scale_cache=vsd,
                                         scaled_kv=True, workspace=workspace)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("hkv,groups,batch,max_len", [
    (8, 4, 1, 40000),   # 157 chunks of one sequence: 10 merge rounds per chunk group
    (8, 4, 3, 9000),
    (8, 1, 2, 12000),   # G = 1: 16 chunk groups
    (8, 3, 2, 7000),    # G = 3: 5 chunk groups, 32 idle threads
    (2, 16, 2, 10000),  # G = 16: one chunk group, 4 outputs per thread in the wave merge
])
def test_many_chunks_merge(hkv, groups, batch, max_len):
    require_gpu()
    q, k, v, ks, vs, tables, lens = _case(20261201 + hkv * 100 + groups, batch, hkv, groups, max_len)
    scale = 128 ** -0.5
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens, scale, k_scale_cache=ks, v_scale_cache=vs)
    for split in (256, 0):  # forced 256-token chunks, then the automatic choice
        set_decode_overrides(path="split", split_tokens=split)
        got = _run(q, k, v, ks, vs, tables, lens, scale)
        assert_decode_close(got, want, label=f"split={split} hkv={hkv} G={groups} B={batch}")


def test_short_and_empty_chunks():
    """Last chunks of 1 token, empty sequences, and chunks whose every page is a hole."""

    require_gpu()
    q, k, v, ks, vs, tables, lens = _case(20261202, 6, 8, 4, 4096, holes=0.0)
    lens[:] = torch.tensor([4096, 257, 256, 1, 0, 2049], dtype=torch.int32)
    tables[0, 4:8] = -1   # with 256-token chunks, chunks 4..7 of sequence 0 attend nothing
    tables[5, 1] = -1
    scale = 0.07
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens, scale, k_scale_cache=ks, v_scale_cache=vs)
    for split in (256, 512, 0):
        set_decode_overrides(path="split", split_tokens=split)
        got = _run(q, k, v, ks, vs, tables, lens, scale)
        assert torch.all(got[4] == 0), "an empty sequence must output zeros"
        assert_decode_close(got, want, label=f"short chunks split={split}")


def test_garbage_workspace_needs_no_clearing():
    """Arbitrary workspace bytes (random, all ones, a streaming call's leftovers) change nothing."""

    require_gpu()
    from prism_infer.ops.paged_decode import decode_workspace_bytes

    q, k, v, ks, vs, tables, lens = _case(20261203, 2, 8, 4, 6000)
    scale = 128 ** -0.5
    set_decode_overrides(path="split", split_tokens=256)
    qd, kd, _, _, _, td, _ = _to_gpu(q, k, v, ks, vs, tables, lens)
    need = decode_workspace_bytes(qd, kd, td)
    assert need > 0
    dev = torch.device("cuda")
    clean = torch.zeros(need + (1 << 20), dtype=torch.uint8, device=dev)
    want_bits = _run(q, k, v, ks, vs, tables, lens, scale, workspace=clean)
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens, scale, k_scale_cache=ks, v_scale_cache=vs)
    assert_decode_close(want_bits, want, label="clean workspace")

    g = torch.Generator(device="cpu").manual_seed(5)
    random_ws = torch.randint(0, 256, (need + (1 << 20),), generator=g, dtype=torch.uint8).to(dev)
    ones_ws = torch.full((need + (1 << 20),), 0xFF, dtype=torch.uint8, device=dev)
    for label, ws in (("random", random_ws), ("0xff", ones_ws)):
        for rep in range(2):  # the second call runs on the counters the first one left
            got = _run(q, k, v, ks, vs, tables, lens, scale, workspace=ws)
            assert torch.equal(got, want_bits), f"{label} workspace, call {rep}"

    # a streaming call of another geometry on the same workspace, then split again
    from prism_infer import workloads
    w = workloads.decode_mixed(dev)
    stream_need = decode_workspace_bytes(w.q, w.k_cache, w.block_tables)
    shared = torch.full((max(stream_need, need) + (1 << 20),), 0x5A, dtype=torch.uint8, device=dev)
    from prism_infer.ops.paged_decode import _launch_paged_decode_attention
    set_decode_overrides(path="stream")
    _launch_paged_decode_attention(w.q, w.k_cache, w.v_cache, w.block_tables, w.context_lens, w.scale,
                                   w.max_context_len, k_scale_cache=w.k_scale, v_scale_cache=w.v_scale,
                                   scaled_kv=True, workspace=shared)
    torch.cuda.synchronize()
    set_decode_overrides(path="split", split_tokens=256)
    got = _run(q, k, v, ks, vs, tables, lens, scale, workspace=shared)
    assert torch.equal(got, want_bits), "split call after a streaming call on the same workspace"
