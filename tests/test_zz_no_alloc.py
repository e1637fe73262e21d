"""The allocation-free decode entry point against the workspace one, through the C ABI.

prism_paged_decode_noalloc (no counterpart in the reference) must give the
same output as prism_paged_decode with a caller workspace, bit for bit (the
same kernels run on the same inputs), on two calls in a row where the second
has a smaller input, so that state the first call left in the shared
scratch (a plan for another geometry, merge counters) cannot leak into the
second.  It must also reject a geometry whose workspace exceeds its 64 MiB
scratch, and it must not allocate device memory through torch.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from _helpers import require_gpu

pytestmark = pytest.mark.gpu


def _args(w, out):
    from prism_infer import _native

    n = _native
    return [
        w.q.data_ptr(), n.dtype_code(w.q.dtype), n.strides(w.q),
        w.k_cache.data_ptr(), w.v_cache.data_ptr(), n.dtype_code(w.k_cache.dtype),
        n.strides(w.k_cache), n.strides(w.v_cache),
        w.k_scale.data_ptr(), w.v_scale.data_ptr(), n.strides(w.k_scale), n.strides(w.v_scale),
        w.block_tables.data_ptr(), n.strides(w.block_tables),
        w.context_lens.data_ptr(), w.max_context_len.data_ptr(),
        out.data_ptr(), n.strides(out),
        w.batch, w.q.shape[1], w.k_cache.shape[2], w.q.shape[2], w.k_cache.shape[1], w.k_cache.shape[0],
        w.block_tables.shape[1], ctypes.c_float(w.scale),
    ]


def _with_workspace(w):
    from prism_infer import _native
    from prism_infer.ops.paged_decode import decode_workspace_bytes

    lib = _native.lib()
    out = torch.full_like(w.q, float("nan"))
    nbytes = decode_workspace_bytes(w.q, w.k_cache, w.block_tables)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=w.q.device)
    status = lib.prism_paged_decode(*_args(w, out), ws.data_ptr(), nbytes, _native.stream_handle(w.q.device))
    _native.check(status, "prism_paged_decode")
    return out


def _no_alloc(w):
    from prism_infer import _native

    lib = _native.lib()
    out = torch.full_like(w.q, float("nan"))
    torch.cuda.synchronize()
    before = torch.cuda.memory_stats().get("allocation.all.allocated", 0)
    status = lib.prism_paged_decode_noalloc(*_args(w, out), _native.stream_handle(w.q.device))
    torch.cuda.synchronize()
    after = torch.cuda.memory_stats().get("allocation.all.allocated", 0)
    _native.check(status, "prism_paged_decode_noalloc")
    assert after == before, "the allocation-free entry point allocated through torch"
    return out


def test_no_alloc_matches_workspace_entry_point_twice():
    require_gpu()
    from prism_infer import workloads

    dev = torch.device("cuda", 0)
    big = workloads.decode_mixed(dev)  # B = 64, streaming kernel, shared prefix
    small = workloads.decode_qwen_vl(dev)  # B = 1, per-split kernel, smaller input
    for w, label in ((big, "B=64 mixed"), (small, "B=1 1800 tokens"), (big, "B=64 mixed again")):
        want = _with_workspace(w)
        got = _no_alloc(w)
        print(f"[{label}] max|d| = {float((got.float() - want.float()).abs().max()):.3e}", flush=True)
        assert torch.isfinite(got).all(), label
        assert torch.equal(got, want), label


def test_no_alloc_rejects_oversized_geometry():
    require_gpu()
    from prism_infer import _native, workloads

    w = workloads.decode_single(torch.device("cuda", 0))
    lib = _native.lib()
    out = torch.empty_like(w.q)
    args = _args(w, out)
    # pretend 1024 sequences of 128 query heads over a 512-page table: about
    # 81 MiB of streaming partials, beyond the 64 MiB scratch (the call is
    # rejected before anything is launched, so the small tensors are never read)
    need = lib.prism_paged_decode_workspace_bytes(1024, 128, 8, 128, 256, 512, 3)
    assert need > 64 << 20
    args[18] = 1024            # batch
    args[19] = 128             # num_heads
    args[24] = 512             # max_blocks_per_seq
    status = lib.prism_paged_decode_noalloc(*args, _native.stream_handle(w.q.device))
    assert status != 0
    assert b"64" in lib.prism_last_error() or b"67108864" in lib.prism_last_error()


def test_no_alloc_refuses_an_overlapping_call_on_another_stream():
    """The scratch is shared per GPU: a call on stream B while stream A's call is still queued is refused
    (PRISM_ERR_BUSY, nothing launched), a call on the same stream is accepted, and once A's call has
    finished B's call runs and gives the workspace entry point's output."""

    require_gpu()
    from prism_infer import _native, workloads

    dev = torch.device("cuda", 0)
    w = workloads.decode_mixed(dev)
    want = _with_workspace(w)
    lib = _native.lib()
    stream_a = torch.cuda.Stream(dev)
    stream_b = torch.cuda.Stream(dev)
    out_a = torch.full_like(w.q, float("nan"))
    out_b = torch.full_like(w.q, float("nan"))
    torch.cuda.synchronize()
    with torch.cuda.stream(stream_a):
        torch.cuda._sleep(200_000_000)  # keeps A's decode queued for tens of milliseconds
        status_a = lib.prism_paged_decode_noalloc(*_args(w, out_a), stream_a.cuda_stream)
        status_a2 = lib.prism_paged_decode_noalloc(*_args(w, out_a), stream_a.cuda_stream)
    status_b = lib.prism_paged_decode_noalloc(*_args(w, out_b), stream_b.cuda_stream)
    message = lib.prism_last_error()
    torch.cuda.synchronize()
    assert status_a == 0 and status_a2 == 0, "calls on one stream are ordered by it"
    assert status_b == -4, f"expected PRISM_ERR_BUSY, got {status_b}"
    assert b"in use" in message
    assert bool(torch.isnan(out_b).all()), "the refused call launched nothing"
    assert torch.equal(out_a, want)
    status_b = lib.prism_paged_decode_noalloc(*_args(w, out_b), stream_b.cuda_stream)
    torch.cuda.synchronize()
    assert status_b == 0
    assert torch.equal(out_b, want)
