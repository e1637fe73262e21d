"""The drop-in boundary without a GPU: C-ABI exports, contract errors, no fallback.

* ``libprism_mi355x.so`` loads (no GPU call is made) and exports every entry
  point ``include/prism_kv.h`` declares, with the ABI version the binding expects;
  the ctypes binding lists exactly those symbols.
* The Python signatures match the reference's (prism_infer/ops/kv_cache_store.py:419-427,
  ops/paged_decode.py:443-455, ops/kv_compaction.py:93-97) and the module flags
  ``HAS_TRITON`` / ``HAS_HIP_KERNELS`` exist.
* Contract violations raise ``ValueError`` with the messages the reference's
  tests match (tests/test_scaled_fp8_kv_cache.py:188-219: "provided together",
  "shape must equal", "torch.float32"; tests/test_paged_decode_kernel.py:346-356:
  "dtype mismatch"), checked on CPU tensors before any device work.
* Valid CPU tensors: the store and compaction take their own torch branch
  (pinned in tests/test_cpu_ops.py); decode raises ``RuntimeError``, as the
  reference's Triton-only decode does.
"""

from __future__ import annotations

import ctypes
import inspect
import re
from pathlib import Path

import pytest
import torch

from prism_infer import _native
from prism_infer.ops import kv_cache_store, kv_compaction, paged_decode
from prism_infer.ops.kv_cache_store import store_kvcache
from prism_infer.ops.kv_compaction import compact_kv_slots
from prism_infer.ops.paged_decode import paged_decode_attention

HEADER = Path(__file__).resolve().parents[1] / "include" / "prism_kv.h"
FP8 = torch.float8_e4m3fn


@pytest.fixture(scope="module")
def lib():
    if not _native.is_built():
        import sys

        sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "prism-infer_amd"))
        import build_native

        build_native.build()
    return _native.lib()


def _declared_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(prism_[a-z0-9_]+)\s*\(", text, flags=re.M)


def test_library_exports_every_declared_symbol(lib):
    names = _declared_symbols()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), f"{name} declared in prism_kv.h but not exported"
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)
    assert sorted(names) == sorted(_native.SIGNATURES), "ctypes binding and header disagree"


def test_abi_version_and_error_string(lib):
    assert lib.prism_abi_version() == _native.ABI_VERSION
    assert isinstance(lib.prism_last_error(), bytes)


def test_workspace_sizing_without_a_device(lib):
    # pure host arithmetic: empty batch needs nothing, bad geometry reports -1
    assert lib.prism_compact_slots_workspace_bytes(2, 1024, 2048, 0) >= 0
    assert lib.prism_compact_slots_workspace_bytes(2, 1024, 2048, 300) >= 2 * 300 * 2048
    assert lib.prism_compact_slots_workspace_bytes(-1, 1, 1, 1) < 0


def test_reference_signatures():
    assert list(inspect.signature(store_kvcache).parameters) == [
        "key", "value", "k_cache", "v_cache", "slot_mapping", "k_scale_cache", "v_scale_cache"]
    params = inspect.signature(paged_decode_attention).parameters
    assert list(params) == ["q", "k_cache", "v_cache", "block_tables", "context_lens", "scale",
                            "k_scale_cache", "v_scale_cache", "max_context_len", "block_n"]
    assert params["block_n"].default == 32
    assert all(params[n].kind is inspect.Parameter.KEYWORD_ONLY
               for n in ("k_scale_cache", "v_scale_cache", "max_context_len", "block_n"))
    assert list(inspect.signature(compact_kv_slots).parameters) == ["cache", "source_slots", "destination_slots"]
    for module in (kv_cache_store, paged_decode, kv_compaction):
        assert isinstance(module.HAS_TRITON, bool) and module.HAS_TRITON == module.HAS_HIP_KERNELS


def _store_args():
    key = torch.randn(1, 2, 8)
    value = torch.randn_like(key)
    k_cache = torch.empty(1, 4, 2, 8, dtype=FP8)
    v_cache = torch.empty_like(k_cache)
    scales = torch.empty(1, 4, 2, dtype=torch.float32)
    slots = torch.tensor([0], dtype=torch.int32)
    return key, value, k_cache, v_cache, slots, scales


def test_store_contract_messages_match_the_reference():
    key, value, k_cache, v_cache, slots, scales = _store_args()
    with pytest.raises(ValueError, match="provided together"):
        store_kvcache(key, value, k_cache, v_cache, slots, scales, None)
    with pytest.raises(ValueError, match="shape must equal"):
        store_kvcache(key, value, k_cache, v_cache, slots, scales[:, :, :1], scales[:, :, :1])
    with pytest.raises(ValueError, match="torch.float32"):
        store_kvcache(key, value, k_cache, v_cache, slots, scales.half(), scales.half())
    with pytest.raises(ValueError, match="one flat slot per input token"):
        store_kvcache(key, value, k_cache, v_cache, torch.tensor([0, 1], dtype=torch.int32), scales, scales)
    with pytest.raises(ValueError, match="FP8"):
        store_kvcache(key, value, k_cache.float(), v_cache.float(), slots, scales, scales)


def test_store_on_cpu_tensors_writes_the_cache():
    key, value, k_cache, v_cache, slots, scales = _store_args()
    v_scales = scales.clone()
    store_kvcache(key, value, k_cache, v_cache, slots, scales, v_scales)
    assert bool((scales.view(-1, scales.shape[-1])[slots.long()] > 0).all())


def _decode_args():
    q = torch.randn(2, 4, 8, dtype=torch.bfloat16)
    k = torch.zeros(3, 4, 2, 8, dtype=FP8)
    v = torch.zeros_like(k)
    ks = torch.ones(3, 4, 2)
    vs = torch.ones(3, 4, 2)
    tables = torch.zeros(2, 2, dtype=torch.int32)
    lens = torch.tensor([3, 5], dtype=torch.int32)
    return q, k, v, tables, lens, ks, vs


def test_decode_contract_messages_match_the_reference():
    q, k, v, tables, lens, ks, vs = _decode_args()
    with pytest.raises(ValueError, match="dtype mismatch"):
        paged_decode_attention(q, k, v.view(torch.uint8).to(torch.bfloat16), tables, lens, 0.3)
    with pytest.raises(ValueError, match="provided together"):
        paged_decode_attention(q, k, v, tables, lens, 0.3, k_scale_cache=ks)
    with pytest.raises(ValueError, match="shape must equal"):
        paged_decode_attention(q, k, v, tables, lens, 0.3, k_scale_cache=ks[:, :2], v_scale_cache=vs[:, :2])
    with pytest.raises(ValueError, match="torch.float32"):
        paged_decode_attention(q, k, v, tables, lens, 0.3, k_scale_cache=ks.half(), v_scale_cache=vs.half())
    with pytest.raises(ValueError, match="power of two"):
        paged_decode_attention(q, k, v, tables, lens, 0.3, k_scale_cache=ks, v_scale_cache=vs, block_n=24)
    with pytest.raises(ValueError, match="torch.int32"):
        paged_decode_attention(q, k, v, tables.long(), lens, 0.3, k_scale_cache=ks, v_scale_cache=vs)
    with pytest.raises(ValueError, match="divisible"):
        paged_decode_attention(q[:, :3], k, v, tables, lens, 0.3, k_scale_cache=ks, v_scale_cache=vs)
    with pytest.raises(ValueError, match="cover q batch"):
        paged_decode_attention(q, k, v, tables[:1], lens, 0.3, k_scale_cache=ks, v_scale_cache=vs)
    with pytest.raises(ValueError, match="FP8"):
        paged_decode_attention(q, k.float(), v.float(), tables, lens, 0.3, k_scale_cache=ks, v_scale_cache=vs)


def test_decode_has_no_cpu_fallback():
    q, k, v, tables, lens, ks, vs = _decode_args()
    with pytest.raises(RuntimeError, match="no CPU fallback|requires GPU|not built|cannot load"):
        paged_decode_attention(q, k, v, tables, lens, 0.3, k_scale_cache=ks, v_scale_cache=vs)


def test_omitted_max_context_len_bounds_nothing():
    """The omitted bound: the reference's context_lens.max() is at least every
    sequence's length, so it never clips; the cached scalar bounds nothing
    either, is int32 of one element on the lengths' device, and is reused."""

    lens = torch.tensor([0, 7, 4096, 3], dtype=torch.int32)
    bound = paged_decode._no_context_bound(lens)
    assert bound.dtype == torch.int32 and bound.numel() == 1 and bound.device == lens.device
    assert int(bound) == 2**31 - 1 and int(bound) >= int(lens.max())
    assert paged_decode._no_context_bound(lens[:2]) is bound
    with pytest.raises(RuntimeError):  # torch's empty-reduction error, as in the reference
        paged_decode._no_context_bound(lens[:0])


def test_compaction_contract_and_cpu_branch():
    cache = torch.zeros(2, 1, 16, 2, 8, dtype=FP8)
    src = torch.tensor([1, 2])
    with pytest.raises(ValueError, match="at least one"):
        compact_kv_slots(cache, src[:0], src[:0])
    with pytest.raises(ValueError, match="shapes must match"):
        compact_kv_slots(cache, src, src[:1])
    with pytest.raises(ValueError, match="torch.long"):
        compact_kv_slots(cache, src.int(), src.int())
    with pytest.raises(ValueError, match=r"\[kv, layers, slots"):
        compact_kv_slots(cache[0, 0], src, src)
    cache.view(torch.uint8)[:, :, 1:3] = 7
    compact_kv_slots(cache, src, torch.tensor([3, 4]))
    assert bool((cache.view(torch.uint8)[:, :, 3:5] == 7).all())


def test_decode_overrides_round_trip():
    """The family overrides are process state set through the C ABI (no GPU needed)."""

    from prism_infer.ops.paged_decode import get_decode_overrides, set_decode_overrides

    set_decode_overrides(path="split", split_tokens=64, share=False)
    assert get_decode_overrides() == ("split", 64, False)
    set_decode_overrides()
    assert get_decode_overrides() == ("auto", 0, True)
    with pytest.raises(ValueError):
        set_decode_overrides(path="fast")
    with pytest.raises(ValueError):
        set_decode_overrides(split_tokens=-1)
