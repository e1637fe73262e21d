"""GPU tests of the streaming decode's plan slots.

The streaming kernel checks, in every workgroup, the plan left in the
workspace by an earlier call (two slots behind a plan word) against its own
metadata; when it differs one workgroup rebuilds the other slot and publishes
it while the rest wait.  These cases drive every branch of that selection on
one workspace:

- metadata alternating between two sets (each call rebuilds into the slot the
  previous call did not use), then repeated (no rebuild): every output equals
  the first output for the same metadata bit for bit, and the two sets match
  the float64 oracle of prism_infer/ops/paged_decode.py:83-180 within the
  decode tolerance of tests/test_scaled_fp8_kv_cache.py:470-472;
- the plan built on its own (stage 3) and then used by the decode kernel
  (stage 1) gives the same bits as the one-launch call;
- a workspace whose plan word carries the building bit with a foreign tag
  (left by an interrupted call, or arbitrary bytes) is rebuilt, not waited on.
"""

from __future__ import annotations

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


def _case():
    g = torch.Generator().manual_seed(20261202)
    batch, width, pool = 48, 12, 600
    q = torch.randn(batch, 32, 128, generator=g).to(torch.bfloat16)
    k, ks = _quantize(torch.randn(pool, 256, 8, 128, generator=g).to(torch.bfloat16))
    v, vs = _quantize(torch.randn(pool, 256, 8, 128, generator=g).to(torch.bfloat16))
    tables = torch.randperm(pool, generator=g)[: batch * width].to(torch.int32).view(batch, width).clone()
    tables[1:20:2, :4] = tables[0, :4]  # a prefix group of 10 sharing 4 pages
    lens_a = torch.randint(1500, width * 256, (batch,), generator=g, dtype=torch.int32)
    lens_b = lens_a.clone()
    lens_b[::3] -= 700                   # different tile counts and sharing lengths
    lens_b[1] = 500                      # a group member below the shared pages
    return q, k, v, ks, vs, tables, lens_a, lens_b


def test_alternating_metadata_on_one_workspace():
    require_gpu()
    from prism_infer.ops.paged_decode import _launch_paged_decode_attention, decode_workspace_bytes

    set_decode_overrides(path="stream")
    dev = torch.device("cuda")
    q, k, v, ks, vs, tables, lens_a, lens_b = _case()
    to = lambda t: t.view(torch.uint8).to(dev).view(FP8) if t.dtype == FP8 else t.to(dev)  # noqa: E731
    qd, kd, vd, ksd, vsd, td = map(to, (q, k, v, ks, vs, tables))
    lens_dev = {"a": to(lens_a), "b": to(lens_b)}
    mx = torch.tensor([tables.shape[1] * 256], dtype=torch.int32, device=dev)
    ws = torch.full((decode_workspace_bytes(qd, kd, td),), 0xFF, dtype=torch.uint8, device=dev)
    scale = 128 ** -0.5

    def run(which, stage=0):
        out = _launch_paged_decode_attention(qd, kd, vd, td, lens_dev[which], scale, mx, k_scale_cache=ksd,
                                             v_scale_cache=vsd, scaled_kv=True, workspace=ws, stage=stage)
        torch.cuda.synchronize()
        return out.cpu()

    first = {"a": run("a"), "b": run("b")}
    for which in ("a", "b"):
        lens = lens_a if which == "a" else lens_b
        want = oracle.decode_kernel_semantics(q, k, v, tables, lens, scale, k_scale_cache=ks, v_scale_cache=vs,
                                              compute_dtype=torch.float32)
        assert_decode_close(first[which], want, label=f"metadata {which}")
    for rep, which in enumerate("abababaa"):  # slot ping-pong, then a reused plan
        assert torch.equal(run(which), first[which]), f"call {rep} ({which})"
    # the plan on its own, then the decode kernel on it
    run("b", stage=3)
    assert torch.equal(run("b", stage=1), first["b"]), "stage 3 then stage 1"


@pytest.mark.parametrize("fill", [0xFF, 0x5A, 0x00])
def test_stale_building_word_is_rebuilt(fill):
    """A plan word with the building bit and any tag but this call's own."""

    require_gpu()
    from prism_infer.ops.paged_decode import _launch_paged_decode_attention, decode_workspace_bytes

    set_decode_overrides(path="stream")
    dev = torch.device("cuda")
    q, k, v, ks, vs, tables, lens_a, _ = _case()
    to = lambda t: t.view(torch.uint8).to(dev).view(FP8) if t.dtype == FP8 else t.to(dev)  # noqa: E731
    qd, kd, vd, ksd, vsd, td, ld = map(to, (q, k, v, ks, vs, tables, lens_a))
    mx = torch.tensor([tables.shape[1] * 256], dtype=torch.int32, device=dev)
    ws = torch.full((decode_workspace_bytes(qd, kd, td),), fill, dtype=torch.uint8, device=dev)
    word = ws[:8].view(torch.int64)
    word.fill_((0x7FFF0000 << 32) | 2 | 1)  # building, slot 1, a tag no call of this process has used yet
    out = _launch_paged_decode_attention(qd, kd, vd, td, ld, 128 ** -0.5, mx, k_scale_cache=ksd, v_scale_cache=vsd,
                                         scaled_kv=True, workspace=ws)
    torch.cuda.synchronize()
    want = oracle.decode_kernel_semantics(q, k, v, tables, lens_a, 128 ** -0.5, k_scale_cache=ks, v_scale_cache=vs,
                                          compute_dtype=torch.float32)
    assert_decode_close(out.cpu(), want, label=f"stale building word, fill {fill:#x}")
    w = int(word.item())
    assert (w & 2) == 0, "the plan word is published"


def test_plan_wait_give_up_is_loud_and_rebuilt():
    """Workgroups that stop waiting for a plan build leave NaN rows, and the next call rebuilds.

    The wait limit is set to 0 polls from the host, so every workgroup that
    finds another one building gives up at once (all kernels still exit).  The
    give-up is counted in the plan header (int 2 of the workspace); the next
    call with the normal limit rebuilds the plan, zeroing the completion
    counters the abandoned call left part-way, and its output is the same bits
    as a call on a fresh workspace.
    """

    require_gpu()
    from prism_infer import _native
    from prism_infer.ops.paged_decode import _launch_paged_decode_attention, decode_workspace_bytes

    set_decode_overrides(path="stream")
    lib = _native.lib()
    dev = torch.device("cuda")
    q, k, v, ks, vs, tables, lens_a, lens_b = _case()
    to = lambda t: t.view(torch.uint8).to(dev).view(FP8) if t.dtype == FP8 else t.to(dev)  # noqa: E731
    qd, kd, vd, ksd, vsd, td = map(to, (q, k, v, ks, vs, tables))
    lens_dev = {"a": to(lens_a), "b": to(lens_b)}
    mx = torch.tensor([tables.shape[1] * 256], dtype=torch.int32, device=dev)
    nbytes = decode_workspace_bytes(qd, kd, td)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)

    def run(which, workspace):
        out = _launch_paged_decode_attention(qd, kd, vd, td, lens_dev[which], 128 ** -0.5, mx, k_scale_cache=ksd,
                                             v_scale_cache=vsd, scaled_kv=True, workspace=workspace)
        torch.cuda.synchronize()
        return out.cpu()

    fresh_b = run("b", torch.zeros(nbytes, dtype=torch.uint8, device=dev))
    run("a", ws)
    default = lib.prism_paged_decode_default_plan_wait_limit()
    previous = lib.prism_paged_decode_set_plan_wait_limit(0)
    try:
        assert previous == default
        abandoned = run("b", ws)  # metadata changed: one workgroup builds, the waiters give up
    finally:
        assert lib.prism_paged_decode_set_plan_wait_limit(default) == 0
    give_ups = int(ws[8:12].view(torch.int32).item())
    print(f"give-ups: {give_ups}, NaN rows: {int(torch.isnan(abandoned.float()).any(-1).any(-1).sum())}", flush=True)
    if give_ups:
        assert bool(torch.isnan(abandoned.float()).any()), "a give-up leaves NaN rows"
    else:
        assert torch.equal(abandoned, fresh_b)
    assert torch.equal(run("b", ws), fresh_b), "rebuilt after the give-up"
    assert int(ws[8:12].view(torch.int32).item()) == 0, "the rebuild clears the give-up count"
    assert torch.equal(run("b", ws), fresh_b), "the rebuilt plan is reused"
    assert lib.prism_paged_decode_set_plan_wait_limit(-1) == -1
