"""GPU parity: HIP slot compaction against the CPU oracle (bit-exact)."""

from __future__ import annotations

import pytest
import torch

import oracle
from _helpers import require_gpu

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


def _compact_both(cache_cpu: torch.Tensor, src: torch.Tensor, dst: torch.Tensor):
    from prism_infer.ops.kv_compaction import compact_kv_slots

    dev = torch.device("cuda")
    if cache_cpu.dtype == FP8:
        gpu = cache_cpu.view(torch.uint8).to(dev).view(FP8)
    else:
        gpu = cache_cpu.to(dev)
    compact_kv_slots(gpu, src.to(dev), dst.to(dev))
    want = cache_cpu.clone()
    oracle.compact_slots(want, src, dst)
    torch.cuda.synchronize()
    got = gpu.view(torch.uint8).cpu() if gpu.dtype == FP8 else gpu.cpu()
    want = want.view(torch.uint8) if want.dtype == FP8 else want
    return got, want


def _bytes_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


def test_reference_fp8_compaction_case():
    """The reference's FP8 compaction case: [2, 2, 8 blocks x 4, 1, 8] with an in-place plan."""

    require_gpu()
    from prism_infer.engine.kv_compaction_plan import plan_in_place

    g = torch.Generator().manual_seed(20260711)
    cache = torch.randn(2, 2, 8, 4, 1, 8, generator=g).to(torch.bfloat16).to(FP8)
    # 10 prompt tokens in blocks (0, 1, 2); keep 6 positions -> compact into blocks (0, 1)
    plan = plan_in_place([0, 1, 2], [0, 1, 4, 5, 8, 9], 4, logical_prompt_len=10)
    src, dst = (torch.tensor(x, dtype=torch.long) for x in (plan.source_slots, plan.destination_slots))
    flat = cache.reshape(2, 2, 32, 1, 8)
    got, want = _compact_both(flat, src, dst)
    assert _bytes_equal(got, want)
    before = flat.view(torch.uint8).index_select(2, src)
    assert torch.equal(got.view(torch.uint8).reshape(2, 2, 32, 1, 8).index_select(2, dst), before)


@pytest.mark.parametrize("in_place", [False, True])
def test_prefix_compaction_config_payload_and_scales(in_place):
    """64 prefixes x 8192 tokens, ~30% visual tokens dropped; payload and fp32 scales, L=1."""

    require_gpu()
    from prism_infer.workloads import compaction_plans

    w = compaction_plans(in_place=in_place)
    slots = w.num_pages * 256
    g = torch.Generator(device="cuda").manual_seed(99)
    payload = torch.randint(0, 256, (2, 1, slots, 8, 128), generator=g, dtype=torch.uint8,
                            device="cuda").cpu().view(FP8)
    scales = torch.rand(2, 1, slots, 8, generator=g, device="cuda").cpu()
    src = torch.tensor([s for p in w.plans for s in p.source_slots], dtype=torch.long)
    dst = torch.tensor([s for p in w.plans for s in p.destination_slots], dtype=torch.long)
    got, want = _compact_both(payload, src, dst)
    assert _bytes_equal(got, want), "payload differs"
    got, want = _compact_both(scales, src, dst)
    assert _bytes_equal(got, want), "scales differ"


def test_overlapping_shift_and_swap_read_before_write():
    require_gpu()
    g = torch.Generator().manual_seed(4)
    cache = torch.randn(2, 3, 64, 5, generator=g)  # 20-byte rows exercise the 4-byte path
    src = torch.arange(1, 64, dtype=torch.long)
    dst = torch.arange(0, 63, dtype=torch.long)
    got, want = _compact_both(cache, src, dst)
    assert _bytes_equal(got, want)
    assert torch.equal(got[:, :, :63], cache[:, :, 1:])
    swap_src = torch.tensor([3, 7, 9, 1], dtype=torch.long)
    swap_dst = torch.tensor([7, 3, 1, 9], dtype=torch.long)
    got, want = _compact_both(cache, swap_src, swap_dst)
    assert _bytes_equal(got, want)
    assert torch.equal(got[:, :, 7], cache[:, :, 3]) and torch.equal(got[:, :, 3], cache[:, :, 7])


def test_identity_and_odd_widths():
    require_gpu()
    cache = torch.arange(2 * 2 * 10 * 3, dtype=torch.uint8).view(2, 2, 10, 3, 1).contiguous()
    src = torch.tensor([0, 2, 3], dtype=torch.long)
    got, want = _compact_both(cache, src, src)  # identity: no change
    assert torch.equal(got, cache)
    got, want = _compact_both(cache, src, torch.tensor([0, 1, 2], dtype=torch.long))
    assert _bytes_equal(got, want)


@pytest.mark.parametrize("vec", ["payload", "scales"])
def test_arbitrary_workspace_contents(vec):
    """The workspace is never cleared: the source tags and the hazard word are compared with the call's
    epoch.  Tags holding every small integer (what recycled memory often holds) and a random hazard word
    give the same bytes as the oracle, on a plan with and without real overlaps."""

    require_gpu()
    from prism_infer import _native

    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(20261212)
    slots = 4096
    shape = (2, 3, slots, 8) if vec == "scales" else (2, 3, slots, 8, 128)
    cache = torch.randint(0, 256, shape, generator=g, dtype=torch.uint8)
    if vec == "payload":
        cache = cache.view(FP8)
    else:
        cache = cache.view(torch.float32)
    lib = _native.lib()
    for overlap in (False, True):
        src = torch.randperm(slots, generator=g)[:1500]
        dst = torch.randperm(slots, generator=g)[:1500] if overlap else torch.arange(2500, 4000)
        if not overlap:
            src = torch.randperm(2500, generator=g)[:1500]
        want = cache.clone()
        oracle.compact_slots(want, src, dst)
        gpu = cache.view(torch.uint8).to(dev).view(cache.dtype)
        rows, vec_bytes = 6, (cache[0, 0, 0].numel() * cache.element_size())
        need = lib.prism_compact_slots_workspace_bytes(rows, slots, vec_bytes, src.numel())
        ws = torch.zeros(need, dtype=torch.uint8, device=dev)
        tags = ws[: slots * 4].view(torch.int32)
        tags.copy_(torch.arange(1, slots + 1, dtype=torch.int32, device=dev) % 4096)  # every small integer
        ws[slots * 4: slots * 4 + 256].copy_(torch.randint(0, 256, (256,), generator=g, dtype=torch.uint8).to(dev))
        s_dev, d_dev = src.to(dev), dst.to(dev)
        status = lib.prism_compact_slots(gpu.data_ptr(), rows, slots, vec_bytes, s_dev.data_ptr(), d_dev.data_ptr(),
                                         src.numel(), ws.data_ptr(), need, _native.stream_handle(dev))
        _native.check(status, "prism_compact_slots")
        torch.cuda.synchronize()
        assert _bytes_equal(gpu.cpu(), want), f"{vec} overlap={overlap}"
