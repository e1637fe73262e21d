"""GPU parity: page-level KV movement (copy-on-write, prefix rows, swaps), bit-exact.

The expectations are the reference runner's own per-block torch copies
(prism_infer/engine/model_runner.py:908-1031) applied on the CPU, and its
lifecycle tests (tests/test_scaled_fp8_kv_cache.py:322-363: payload and scales
move together; swap out then in restores a block).
"""

from __future__ import annotations

import pytest
import torch

from _helpers import require_gpu

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn


def _caches(seed, layers=3, blocks=12, page=16, heads=2, dim=8):
    g = torch.Generator().manual_seed(seed)
    payload = torch.randn(2, layers, blocks, page, heads, dim, generator=g).to(FP8)
    scales = torch.rand(2, layers, blocks, page, heads, generator=g)
    return payload, scales


def _to_gpu(t):
    return t.view(torch.uint8).cuda().view(FP8) if t.dtype == FP8 else t.cuda()


def _bytes(t):
    return t.view(torch.uint8) if t.dtype == FP8 else t


def test_copy_on_write_blocks_payload_and_scales():
    require_gpu()
    from prism_infer.engine.kv_block_ops import copy_kv_blocks

    payload, scales = _caches(1)
    pairs = [(0, 5), (3, 7), (1, 2), (3, 11)]
    want_p, want_s = payload.clone(), scales.clone()
    for s, d in pairs:  # the reference's loop
        want_p[:, :, d].view(torch.uint8).copy_(want_p[:, :, s].view(torch.uint8))
        want_s[:, :, d].copy_(want_s[:, :, s])
    gp, gs = _to_gpu(payload), _to_gpu(scales)
    copy_kv_blocks(gp, pairs, gs)
    assert torch.equal(_bytes(gp).cpu(), _bytes(want_p))
    assert torch.equal(gs.cpu(), want_s)


def test_copy_block_prefix_rows():
    require_gpu()
    from prism_infer.engine.kv_block_ops import copy_kv_block_prefixes

    payload, scales = _caches(2)
    copies = [(4, 9, 16), (6, 1, 5), (2, 3, 1)]
    want_p, want_s = payload.clone(), scales.clone()
    for s, d, n in copies:
        want_p[:, :, d, :n].view(torch.uint8).copy_(want_p[:, :, s, :n].view(torch.uint8))
        want_s[:, :, d, :n].copy_(want_s[:, :, s, :n])
    gp, gs = _to_gpu(payload), _to_gpu(scales)
    copy_kv_block_prefixes(gp, copies, gs)
    assert torch.equal(_bytes(gp).cpu(), _bytes(want_p))
    assert torch.equal(gs.cpu(), want_s)


def test_swap_out_and_in_restore_blocks():
    require_gpu()
    from prism_infer.engine.kv_block_ops import swap_blocks

    payload, scales = _caches(3, blocks=6)
    gp, gs = _to_gpu(payload), _to_gpu(scales)
    cpu_p = torch.zeros(2, 3, 4, 16, 2, 8, dtype=torch.uint8).pin_memory().view(FP8)
    cpu_s = torch.zeros(2, 3, 4, 16, 2).pin_memory()
    swap_blocks(gp, cpu_p, [(0, 0), (5, 3), (2, 1)], "out", gpu_scale_cache=gs, cpu_scale_cache=cpu_s)
    for s, d in [(0, 0), (5, 3), (2, 1)]:
        assert torch.equal(cpu_p[:, :, d].view(torch.uint8), payload[:, :, s].view(torch.uint8))
        assert torch.equal(cpu_s[:, :, d], scales[:, :, s])
    gp[:, :, 4].view(torch.uint8).zero_()
    gs[:, :, 4].zero_()
    swap_blocks(gp, cpu_p, [(3, 4)], "in", gpu_scale_cache=gs, cpu_scale_cache=cpu_s)
    assert torch.equal(_bytes(gp[:, :, 4]).cpu(), payload[:, :, 5].view(torch.uint8))
    assert torch.equal(gs[:, :, 4].cpu(), scales[:, :, 5])
    untouched = [0, 1, 2, 3, 5]
    assert torch.equal(_bytes(gp[:, :, untouched]).cpu(), payload[:, :, untouched].view(torch.uint8))


def test_engine_shape_copy_on_write_and_prefix():
    """36-layer engine shape: 8 kv heads x 128 dims, 256-token pages."""

    require_gpu()
    from prism_infer.engine.kv_block_ops import copy_kv_block_prefixes, copy_kv_blocks

    g = torch.Generator(device="cuda").manual_seed(4)
    gp = torch.randint(0, 255, (2, 36, 24, 256, 8, 128), dtype=torch.uint8, device="cuda", generator=g).view(FP8)
    gs = torch.rand(2, 36, 24, 256, 8, device="cuda", generator=g)
    before_p, before_s = gp.view(torch.uint8).clone(), gs.clone()
    copy_kv_blocks(gp, [(0, 20), (1, 21)], gs)
    copy_kv_block_prefixes(gp, [(2, 22, 100)], gs)
    want_p, want_s = before_p.clone(), before_s.clone()
    want_p[:, :, 20] = before_p[:, :, 0]
    want_p[:, :, 21] = before_p[:, :, 1]
    want_p[:, :, 22, :100] = before_p[:, :, 2, :100]
    want_s[:, :, 20] = before_s[:, :, 0]
    want_s[:, :, 21] = before_s[:, :, 1]
    want_s[:, :, 22, :100] = before_s[:, :, 2, :100]
    assert torch.equal(gp.view(torch.uint8), want_p)
    assert torch.equal(gs, want_s)
