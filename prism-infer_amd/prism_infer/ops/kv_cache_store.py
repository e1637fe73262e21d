"""Physical writes into canonical paged KV-cache storage (MI355X HIP kernels).

Drop-in for prism_infer/ops/kv_cache_store.py: same ``store_kvcache``
signature (:419-427), same contract validation and error messages
(:233-337), same storage semantics (scaled path :81-167 / :205-227, dense
path :58-78 / :228-230).  The work is done by ``prism_kv_store`` in
libprism_mi355x.so.  Differences from the reference, all deliberate:

* CPU tensors take a vectorized torch path of this module's own (the
  reference routes them to a per-token Python loop, :439-476); GPU tensors
  always take the HIP kernels, and a missing native library raises there;
* the scaled path is bit-exact against the eager oracle, including scales
  (the reference's Triton kernel is only checked to 1e-6 relative);
* slots >= the cache's slot count are skipped instead of written out of bounds.
"""

from __future__ import annotations

import torch

from prism_infer import _native
from prism_infer.engine.kv_quantization import (
    FP8_E4M3FN_MAX,
    FP8_E4M3FN_MIN,
    KV_SCALE_DTYPE,
    PER_TOKEN_HEAD_SCALE_FLOOR,
    scale_cache_shape,
)
from prism_infer.observability import profile_region

# "Kernel available" flag.  The reference exports HAS_TRITON for the same
# purpose and its callers/tests import that name, so both are provided.
HAS_HIP_KERNELS = _native.available()
HAS_TRITON = HAS_HIP_KERNELS

KV_TOKEN_HEAD_TENSOR_RANK = 3
SUPPORTED_KV_CACHE_RANKS = (3, 4)
SLOT_MAPPING_TENSOR_RANK = 1


def _float8_cache_dtypes() -> tuple[torch.dtype, ...]:
    return (torch.float8_e4m3fn,) if hasattr(torch, "float8_e4m3fn") else ()


FP8_CACHE_DTYPES = _float8_cache_dtypes()


def is_fp8_cache_tensor(tensor: torch.Tensor) -> bool:
    """Return whether ``tensor`` uses a supported FP8 KV payload dtype."""

    return tensor.dtype in FP8_CACHE_DTYPES


def _validate_store_inputs(key, value, k_cache, v_cache, slot_mapping, k_scale_cache, v_scale_cache) -> bool:
    """Validate the public storage contract and return whether scales are used."""

    _validate_payload_store_inputs(key, value, k_cache, v_cache, slot_mapping)
    return _validate_scale_store_inputs(k_cache, k_scale_cache, v_scale_cache)


def _validate_payload_store_inputs(key, value, k_cache, v_cache, slot_mapping) -> None:
    if (
        key.ndim != KV_TOKEN_HEAD_TENSOR_RANK
        or value.ndim != KV_TOKEN_HEAD_TENSOR_RANK
        or key.shape != value.shape
    ):
        raise ValueError(
            "key/value must have the same [tokens, KV heads, head dim] shape, "
            f"got {list(key.shape)} and {list(value.shape)}"
        )
    if k_cache.shape != v_cache.shape or k_cache.dtype != v_cache.dtype:
        raise ValueError("K/V payload caches must have matching shape and dtype")
    if k_cache.ndim not in SUPPORTED_KV_CACHE_RANKS:
        raise ValueError("K/V payload caches must be [slots, heads, dim] or [blocks, page, heads, dim]")
    if tuple(k_cache.shape[-2:]) != tuple(key.shape[-2:]):
        raise ValueError(
            "input/cache KV head shape mismatch: "
            f"input={list(key.shape[-2:])}, cache={list(k_cache.shape[-2:])}"
        )
    if slot_mapping.ndim != SLOT_MAPPING_TENSOR_RANK or slot_mapping.numel() != key.shape[0]:
        raise ValueError("slot_mapping must contain one flat slot per input token")


def _validate_scale_store_inputs(k_cache, k_scale_cache, v_scale_cache) -> bool:
    if (k_scale_cache is None) != (v_scale_cache is None):
        raise ValueError("K/V scale caches must be provided together")
    if k_scale_cache is None:
        return False
    if not is_fp8_cache_tensor(k_cache):
        raise ValueError("token-head scales require FP8 K/V payload caches")
    expected = scale_cache_shape(k_cache.shape)
    if k_scale_cache.shape != v_scale_cache.shape or tuple(k_scale_cache.shape) != expected:
        raise ValueError(
            "K/V scale cache shape must equal payload shape without head_dim: "
            f"expected={list(expected)}"
        )
    if k_scale_cache.dtype != KV_SCALE_DTYPE or v_scale_cache.dtype != KV_SCALE_DTYPE:
        raise ValueError("K/V scale caches must use torch.float32")
    return True


def _validate_device_store_layout(key, value, k_cache, v_cache, slot_mapping, k_scale_cache, v_scale_cache) -> None:
    """The GPU layout contract (reference :305-337, same messages modulo the backend name)."""

    scales = tuple(t for t in (k_scale_cache, v_scale_cache) if t is not None)
    tensors = (key, value, k_cache, v_cache, slot_mapping, *scales)
    if any(not t.is_cuda for t in tensors):
        raise RuntimeError("MI355X KV store requires all tensors on the GPU (there is no CPU fallback)")
    if any(t.device != key.device for t in tensors[1:]):
        raise RuntimeError("MI355X KV store requires all tensors on the same device")
    if slot_mapping.dtype != torch.int32:
        raise ValueError("MI355X KV store requires torch.int32 slot_mapping")
    head_dim = key.shape[-1]
    if key.stride(-1) != 1 or value.stride(-1) != 1 or key.stride(-2) != head_dim or value.stride(-2) != head_dim:
        raise RuntimeError("MI355X KV store requires contiguous head/dim inputs")
    if not k_cache.is_contiguous() or not v_cache.is_contiguous():
        raise RuntimeError("MI355X KV store requires contiguous KV caches")
    if scales and (not k_scale_cache.is_contiguous() or not v_scale_cache.is_contiguous()):
        raise RuntimeError("MI355X scaled KV store requires contiguous scale caches")
    if key.dtype not in (torch.float32, torch.bfloat16, torch.float16) or key.dtype != value.dtype:
        raise ValueError(f"key/value dtype must be one of float32/bfloat16/float16 and match, got {key.dtype}/{value.dtype}")


def _store_profile_region(scaled: bool, k_cache: torch.Tensor, on_cpu: bool = False) -> str:
    if on_cpu:
        return "attention.kv_store.eager"
    if scaled:
        return "attention.kv_store.hip_scaled_fp8"
    if is_fp8_cache_tensor(k_cache):
        return "attention.kv_store.hip_fp8"
    return "attention.kv_store.hip"


def _last_writer_rows(slot_mapping: torch.Tensor, num_slots: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(token rows, slots) to write: slots < 0 are skipped and, for a slot named
    by several tokens, only the last token is kept (the reference's loop writes
    tokens in order, so the last one is what the slot holds afterwards)."""

    slots = slot_mapping.to(torch.long)
    rows = torch.nonzero(slots >= 0).flatten()
    slots = slots[rows]
    if slots.numel() and int(slots.max()) >= num_slots:
        bad = int(slots.max())
        raise IndexError(f"slot {bad} is out of range for a KV cache of {num_slots} slots")
    if slots.numel() > 1:
        unique, inverse = torch.unique(slots, return_inverse=True)
        last = torch.full((unique.numel(),), -1, dtype=torch.long)
        last.scatter_reduce_(0, inverse, rows, reduce="amax")
        rows, slots = last, unique
    return rows, slots


def _quantize_rows(x: torch.Tensor, cache_dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """[n, heads, dim] -> (E4M3FN payload, fp32 scale per (row, head)).

    scale = max(amax|x| / 448, floor), payload = RNE(clamp(x / scale, +-448));
    the quotient is an IEEE fp32 division, as in the reference's loop."""

    xf = x.float()
    scale = torch.clamp(xf.abs().amax(dim=-1) / FP8_E4M3FN_MAX, min=PER_TOKEN_HEAD_SCALE_FLOOR)
    payload = torch.clamp(xf / scale.unsqueeze(-1), min=FP8_E4M3FN_MIN, max=FP8_E4M3FN_MAX).to(cache_dtype)
    return payload, scale


def _store_kvcache_cpu(key, value, k_cache, v_cache, slot_mapping, k_scale_cache, v_scale_cache) -> None:
    """Host-tensor store: the reference's eager semantics (:183-230), vectorized
    over tokens. Payload rows and scales are written with index_copy_ on flat
    [slots, heads, dim] / [slots, heads] views of the caches."""

    caches = tuple(t for t in (k_cache, v_cache, k_scale_cache, v_scale_cache) if t is not None)
    if not all(t.is_contiguous() for t in caches):
        raise RuntimeError("KV store requires contiguous KV and scale caches")
    heads, dim = key.shape[-2], key.shape[-1]
    flat_k = k_cache.view(-1, heads, dim)
    flat_v = v_cache.view(-1, heads, dim)
    rows, slots = _last_writer_rows(slot_mapping, flat_k.shape[0])
    if rows.numel() == 0:
        return
    k_rows = key.index_select(0, rows)
    v_rows = value.index_select(0, rows)
    if k_scale_cache is None:
        _index_copy_bytes(flat_k, slots, k_rows.to(k_cache.dtype))
        _index_copy_bytes(flat_v, slots, v_rows.to(v_cache.dtype))
        return
    k_payload, k_scale = _quantize_rows(k_rows, k_cache.dtype)
    v_payload, v_scale = _quantize_rows(v_rows, v_cache.dtype)
    _index_copy_bytes(flat_k, slots, k_payload)
    _index_copy_bytes(flat_v, slots, v_payload)
    _index_copy_bytes(k_scale_cache.view(-1, heads), slots, k_scale)
    _index_copy_bytes(v_scale_cache.view(-1, heads), slots, v_scale)


def _index_copy_bytes(dst: torch.Tensor, index: torch.Tensor, rows: torch.Tensor) -> None:
    """dst[index[i]] = rows[i], moved as raw bytes (exact for every dtype,
    NaN payloads included)."""

    as_bytes = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[dst.element_size()]
    dst.view(as_bytes).index_copy_(0, index, rows.contiguous().view(as_bytes))


def store_kvcache(
    key: torch.Tensor,
    value: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    k_scale_cache: torch.Tensor | None = None,
    v_scale_cache: torch.Tensor | None = None,
) -> None:
    """Write current K/V values into canonical paged KV-cache slots (in place)."""

    scaled = _validate_store_inputs(key, value, k_cache, v_cache, slot_mapping, k_scale_cache, v_scale_cache)
    tensors = (key, value, k_cache, v_cache, slot_mapping, k_scale_cache, v_scale_cache)
    if not any(t is not None and t.is_cuda for t in tensors):
        with profile_region(
            _store_profile_region(scaled, k_cache, on_cpu=True),
            metadata={"cache_dtype": str(k_cache.dtype), "tokens": key.shape[0]},
        ):
            _store_kvcache_cpu(key, value, k_cache, v_cache, slot_mapping, k_scale_cache, v_scale_cache)
        return
    _validate_device_store_layout(key, value, k_cache, v_cache, slot_mapping, k_scale_cache, v_scale_cache)
    num_tokens, num_heads, head_dim = key.shape
    num_slots = k_cache.numel() // (num_heads * head_dim) if k_cache.numel() else 0
    lib = _native.device_lib(key.device)
    with profile_region(
        _store_profile_region(scaled, k_cache),
        metadata={"cache_dtype": str(k_cache.dtype), "tokens": num_tokens},
    ), torch.cuda.device(key.device):
        status = lib.prism_kv_store(
            key.data_ptr(), value.data_ptr(), _native.dtype_code(key.dtype),
            _native.strides(key), _native.strides(value),
            k_cache.data_ptr(), v_cache.data_ptr(), _native.dtype_code(k_cache.dtype),
            k_scale_cache.data_ptr() if scaled else None,
            v_scale_cache.data_ptr() if scaled else None,
            slot_mapping.data_ptr(), num_tokens, num_heads, head_dim, num_slots,
            _native.stream_handle(key.device),
        )
    _native.check(status, "store_kvcache")


__all__ = [
    "FP8_CACHE_DTYPES",
    "FP8_E4M3FN_MAX",
    "FP8_E4M3FN_MIN",
    "HAS_HIP_KERNELS",
    "HAS_TRITON",
    "PER_TOKEN_HEAD_SCALE_FLOOR",
    "is_fp8_cache_tensor",
    "store_kvcache",
]
