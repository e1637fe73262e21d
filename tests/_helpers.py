"""Shared helpers for the parity tests (CPU copies of the touched pages)."""

from __future__ import annotations

import torch


def require_gpu() -> None:
    import pytest

    if not torch.cuda.is_available():
        pytest.skip("needs a GPU")


def compact_to_cpu(w, page_ids: torch.Tensor | None = None):
    """Copy only the pages a workload references to CPU and remap its tables.

    Returns (q, k, v, ks, vs, tables, lens, max_ctx) on CPU, where the caches
    hold just the referenced pages (same bytes) and ``tables`` points into them.
    """

    tables = w.block_tables.cpu().to(torch.int64)
    used = torch.unique(tables[tables >= 0]) if page_ids is None else page_ids
    remap = torch.full((w.k_cache.shape[0],), -1, dtype=torch.int64)
    remap[used] = torch.arange(used.numel())
    new_tables = torch.where(tables >= 0, remap[tables.clamp(min=0)], tables).to(torch.int32)
    idx = used.to(w.k_cache.device)
    k = w.k_cache.index_select(0, idx).cpu() if w.k_cache.dtype != torch.float8_e4m3fn else \
        w.k_cache.view(torch.uint8).index_select(0, idx).cpu().view(torch.float8_e4m3fn)
    v = w.v_cache.index_select(0, idx).cpu() if w.v_cache.dtype != torch.float8_e4m3fn else \
        w.v_cache.view(torch.uint8).index_select(0, idx).cpu().view(torch.float8_e4m3fn)
    ks = w.k_scale.index_select(0, idx).cpu()
    vs = w.v_scale.index_select(0, idx).cpu()
    return (w.q.cpu(), k, v, ks, vs, new_tables, w.context_lens.cpu(), int(w.max_context_len.item()))


def diff_stats(actual: torch.Tensor, expected: torch.Tensor) -> tuple[float, float]:
    d = (actual.float().cpu() - expected.float().cpu()).abs()
    return float(d.max()), float(d.mean())


def assert_decode_close(actual, expected, *, atol=2e-2, rtol=1e-2, mean_tol=2e-3, label="") -> None:
    """Decode tolerance of the scaled-FP8 path: |a-e| <= atol + rtol|e| and mean |a-e| < mean_tol."""

    a = actual.float().cpu()
    e = expected.float().cpu()
    assert a.shape == e.shape, (label, a.shape, e.shape)
    assert torch.isfinite(a).all(), f"{label}: non-finite output"
    err = (a - e).abs()
    bound = atol + rtol * e.abs()
    worst = float((err - bound).max())
    mx, mean = float(err.max()), float(err.mean())
    print(f"[{label}] max|d|={mx:.3e} mean|d|={mean:.3e}", flush=True)
    assert worst <= 0, f"{label}: max|d|={mx:.3e} exceeds atol {atol} + rtol {rtol}|e|"
    assert mean < mean_tol, f"{label}: mean|d|={mean:.3e} >= {mean_tol}"
