"""Python side of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Byte/integer work (fp8 encoding, the scaled store, compaction) runs in the C
restatement ``oracle/kv_oracle.c`` through ctypes; floating-point decode
references are written with torch on CPU.  Reference citations are paths in
the Prism-Infer source tree.
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

ORACLE_DIR = Path(__file__).resolve().parent
_LIB_PATH = ORACLE_DIR / "liboracle.so"
_LIB = None

FP8_E4M3FN_MAX = 448.0  # prism_infer/engine/kv_quantization.py:9
PER_TOKEN_HEAD_SCALE_FLOOR = 1.0e-6  # prism_infer/engine/kv_quantization.py:11

_IN_DTYPE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}

__all__ = [
    "build_oracle",
    "e4m3fn_encode",
    "e4m3fn_encode_bit_range",
    "e4m3fn_decode_table",
    "store_scaled",
    "store_scaled_torch_loop",
    "store_unit",
    "compact_slots",
    "compact_slots_torch",
    "decode_kernel_semantics",
    "decode_reference_qdtype",
    "decode_reference_fp32",
    "decode_bruteforce_f64",
    "dequantize",
    "decode_token_mask",
    "prefill_reference_qdtype",
    "prefill_reference_fp32",
    "prefill_bruteforce_f64",
]


def build_oracle(force: bool = False) -> Path:
    """Compile ``liboracle.so`` with the committed Makefile (gcc, no fast-math)."""

    if force or not _LIB_PATH.exists() or (
        _LIB_PATH.stat().st_mtime < (ORACLE_DIR / "kv_oracle.c").stat().st_mtime
    ):
        subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), "-B" if force else "all"], check=True)
    return _LIB_PATH


def _lib():
    global _LIB
    if _LIB is None:
        if not _LIB_PATH.exists():
            build_oracle()
        lib = ctypes.CDLL(str(_LIB_PATH))
        i64p = ctypes.POINTER(ctypes.c_int64)
        lib.oracle_e4m3fn_from_f32.restype = ctypes.c_uint8
        lib.oracle_e4m3fn_from_f32.argtypes = [ctypes.c_float]
        lib.oracle_e4m3fn_to_f32.restype = ctypes.c_float
        lib.oracle_e4m3fn_to_f32.argtypes = [ctypes.c_uint8]
        lib.oracle_e4m3fn_encode_array.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        lib.oracle_e4m3fn_encode_bit_range.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
        lib.oracle_store_scaled.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, i64p, i64p,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
        ]
        lib.oracle_store_unit.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, i64p, i64p,
            ctypes.c_void_p, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
        ]
        lib.oracle_compact_slots.restype = ctypes.c_int
        lib.oracle_compact_slots.argtypes = [
            ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
        ]
        _LIB = lib
    return _LIB


# --------------------------------------------------------------------------- fp8 codec


def e4m3fn_encode(values: np.ndarray) -> np.ndarray:
    """fp32 -> E4M3FN bytes (RNE; overflow and NaN -> NaN code with sign)."""

    src = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(src.shape, dtype=np.uint8)
    _lib().oracle_e4m3fn_encode_array(src.ctypes.data, out.ctypes.data, src.size)
    return out


def e4m3fn_encode_bit_range(lo: int, hi: int) -> np.ndarray:
    """Encode every fp32 bit pattern in ``[lo, hi)``."""

    out = np.empty(hi - lo, dtype=np.uint8)
    _lib().oracle_e4m3fn_encode_bit_range(lo, hi, out.ctypes.data)
    return out


def e4m3fn_decode_table() -> np.ndarray:
    """All 256 E4M3FN codes decoded to fp32 (NaN codes 0x7F/0xFF -> NaN)."""

    lib = _lib()
    return np.array([lib.oracle_e4m3fn_to_f32(b) for b in range(256)], dtype=np.float32)


# --------------------------------------------------------------------------- store


def _i64(values) -> ctypes.Array:
    return (ctypes.c_int64 * len(values))(*[int(v) for v in values])


def _check_cpu(*tensors: torch.Tensor) -> None:
    for tensor in tensors:
        if tensor.device.type != "cpu":
            raise RuntimeError("the oracle runs on CPU tensors only")


def store_scaled(key, value, k_cache, v_cache, slot_mapping, k_scale_cache, v_scale_cache) -> None:
    """Restates ``_store_kvcache_eager`` scaled branch (ops/kv_cache_store.py:170-227).

    ``k_cache``/``v_cache`` are FP8 (or uint8) tensors of shape [..., H, D],
    contiguous; scale caches fp32 [..., H] contiguous.  Mutates in place.
    """

    _check_cpu(key, value, k_cache, v_cache, slot_mapping, k_scale_cache, v_scale_cache)
    num_tokens, num_heads, head_dim = key.shape
    slots = slot_mapping.to(torch.int32).contiguous()
    kc = k_cache.view(torch.uint8)
    vc = v_cache.view(torch.uint8)
    assert kc.is_contiguous() and vc.is_contiguous()
    assert k_scale_cache.is_contiguous() and v_scale_cache.is_contiguous()
    _lib().oracle_store_scaled(
        key.data_ptr(), value.data_ptr(), _IN_DTYPE[key.dtype],
        _i64(key.stride()), _i64(value.stride()),
        kc.data_ptr(), vc.data_ptr(), k_scale_cache.data_ptr(), v_scale_cache.data_ptr(),
        slots.data_ptr(), num_tokens, num_heads, head_dim, kc.numel() // (num_heads * head_dim),
    )


def store_scaled_torch_loop(key, value, k_cache, v_cache, slot_mapping, k_scale_cache, v_scale_cache) -> None:
    """The reference's CPU store path as it runs: a Python loop over tokens with
    torch ops per token (``_store_kvcache_eager``, ops/kv_cache_store.py:170-227).

    Per token with slot >= 0 and per head: s = max(amax|x| / 448, 1e-6) in
    fp32, payload = clamp(x / s, -448, 448) cast to E4M3FN (torch's RNE cast).
    It is what ``bench.py``'s CPU baseline times for the store; the tests pin
    it to the C restatement above byte for byte.
    """

    _check_cpu(key, value, k_cache, v_cache, slot_mapping, k_scale_cache, v_scale_cache)
    heads, dim = k_cache.shape[-2], k_cache.shape[-1]
    kc = k_cache.view(-1, heads, dim)
    vc = v_cache.view(-1, heads, dim)
    ksc = k_scale_cache.view(-1, heads)
    vsc = v_scale_cache.view(-1, heads)
    slots = slot_mapping.tolist()
    for t, slot in enumerate(slots):
        if slot < 0:
            continue
        for src, payload, scales in ((key[t], kc, ksc), (value[t], vc, vsc)):
            xf = src.float()
            s = (xf.abs().amax(dim=-1) / 448.0).clamp(min=1.0e-6)
            payload[slot] = (xf / s[:, None]).clamp(-448.0, 448.0).to(payload.dtype)
            scales[slot] = s


def store_unit(key, value, k_cache, v_cache, slot_mapping) -> None:
    """Restates the dense branch into FP8 caches (ops/kv_cache_store.py:228-230)."""

    _check_cpu(key, value, k_cache, v_cache, slot_mapping)
    num_tokens, num_heads, head_dim = key.shape
    slots = slot_mapping.to(torch.int32).contiguous()
    kc = k_cache.view(torch.uint8)
    vc = v_cache.view(torch.uint8)
    _lib().oracle_store_unit(
        key.data_ptr(), value.data_ptr(), _IN_DTYPE[key.dtype],
        _i64(key.stride()), _i64(value.stride()),
        kc.data_ptr(), vc.data_ptr(), slots.data_ptr(), num_tokens, num_heads, head_dim,
        kc.numel() // (num_heads * head_dim),
    )


# --------------------------------------------------------------------------- compaction


def compact_slots(cache: torch.Tensor, source_slots: torch.Tensor, destination_slots: torch.Tensor) -> None:
    """Restates ``compact_kv_slots`` (ops/kv_compaction.py:93-112) on raw bytes.

    ``cache``: contiguous [kv, layers, slots, ...]; all reads precede all writes.
    """

    _check_cpu(cache, source_slots, destination_slots)
    if not cache.is_contiguous():
        raise RuntimeError("oracle compaction expects a contiguous cache")
    rows = cache.shape[0] * cache.shape[1]
    num_slots = cache.shape[2]
    vec_bytes = math.prod(cache.shape[3:]) * cache.element_size()
    src = source_slots.to(torch.int64).contiguous()
    dst = destination_slots.to(torch.int64).contiguous()
    raw = cache.view(torch.uint8) if cache.element_size() == 1 else cache.view(-1).view(torch.uint8)
    rc = _lib().oracle_compact_slots(raw.data_ptr(), rows, num_slots, vec_bytes,
                                     src.data_ptr(), dst.data_ptr(), src.numel())
    if rc == -2:
        raise IndexError("compaction slot index out of range")
    if rc != 0:
        raise MemoryError("oracle compaction could not allocate its temporary")


def compact_slots_torch(cache: torch.Tensor, source_slots: torch.Tensor, destination_slots: torch.Tensor) -> None:
    """The library formulation the reference uses for non-FP8 caches (kv_compaction.py:111-112)."""

    retained = cache.index_select(2, source_slots).clone()
    cache.index_copy_(2, destination_slots, retained)


# --------------------------------------------------------------------------- decode


def dequantize(payload: torch.Tensor, scales: torch.Tensor | None, dtype: torch.dtype) -> torch.Tensor:
    """``dequantize_cache_for_attention`` (ops/paged_attention_reference.py:102-122).

    With ``dtype=bfloat16`` the product ``fp8.to(bf16) * scale.to(bf16)`` is
    rounded to bf16 exactly as the reference's CPU path does.
    """

    result = payload.to(dtype)
    if scales is not None:
        result = result * scales.to(dtype).unsqueeze(-1)
    return result


def decode_token_mask(block_row: torch.Tensor, context_len: int, max_context_len: int,
                      page_size: int, num_blocks: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Token validity of the reference kernel (ops/paged_decode.py:95-119).

    A logical token t is attended iff ``t < min(context_len, max_context_len,
    W * page_size)`` and its block id is >= 0.  Block ids >= ``num_blocks`` are
    treated as absent (the reference would read out of bounds; the HIP path
    skips them, and the oracle states the same contract).
    Returns (block ids per token, valid mask) over ``range(W * page_size)``.
    """

    width = block_row.numel()
    capacity = width * page_size
    bound = max(0, min(int(context_len), int(max_context_len), capacity))
    tokens = torch.arange(capacity)
    blocks = block_row.to(torch.int64)[tokens // page_size]
    valid = (tokens < bound) & (blocks >= 0) & (blocks < num_blocks)
    return blocks, valid


def decode_kernel_semantics(q, k_cache, v_cache, block_tables, context_lens, scale, *,
                            k_scale_cache=None, v_scale_cache=None, max_context_len=None,
                            compute_dtype=torch.float64) -> torch.Tensor:
    """Single-query paged attention with the reference kernel's semantics.

    Restates ``_paged_decode_attention_kernel`` (ops/paged_decode.py:83-180):
    kv head ``hq // G``; K and V dequantized in fp32 (``fp8 -> fp32 * scale``,
    :121-139, :150-168); softmax over the valid tokens of
    :func:`decode_token_mask`; output 0 when no token is valid (:173-175).
    The softmax itself is evaluated in ``compute_dtype`` (float64 by default)
    so the result is the exact attention of the dequantized cache.
    Returns a tensor in ``q.dtype``.
    """

    batch, num_heads, head_dim = q.shape
    num_blocks, page_size, num_kv_heads, _ = k_cache.shape
    groups = num_heads // num_kv_heads
    if max_context_len is None:
        max_context_len = int(context_lens[:batch].max().item()) if batch else 0
    out = torch.zeros(batch, num_heads, head_dim, dtype=compute_dtype)
    for b in range(batch):
        blocks, valid = decode_token_mask(block_tables[b], int(context_lens[b]), int(max_context_len),
                                          page_size, num_blocks)
        idx = torch.nonzero(valid).flatten()
        if idx.numel() == 0:
            continue
        blk = blocks[idx]
        off = idx % page_size
        keys = k_cache[blk, off].to(torch.float32)
        values = v_cache[blk, off].to(torch.float32)
        if k_scale_cache is not None:
            keys = keys * k_scale_cache[blk, off].to(torch.float32).unsqueeze(-1)
            values = values * v_scale_cache[blk, off].to(torch.float32).unsqueeze(-1)
        keys = keys.to(compute_dtype).repeat_interleave(groups, dim=1)      # [n, Hq, D]
        values = values.to(compute_dtype).repeat_interleave(groups, dim=1)
        qb = q[b].to(compute_dtype)                                        # [Hq, D]
        scores = torch.einsum("hd,nhd->hn", qb, keys) * scale
        probs = torch.softmax(scores, dim=-1)
        out[b] = torch.einsum("hn,nhd->hd", probs, values)
    return out.to(q.dtype)


def _gather_sequence(cache: torch.Tensor, block_row: torch.Tensor, context_len: int) -> torch.Tensor:
    """``gather_paged_kv_for_sequence`` (ops/paged_attention_reference.py:22-63)."""

    if context_len <= 0:
        raise ValueError(f"context_len must be positive, got {context_len}")
    pieces = []
    remaining = context_len
    page_size = cache.shape[1]
    for block_id in block_row.tolist():
        if remaining <= 0 or block_id < 0:
            break
        if block_id >= cache.shape[0]:
            raise RuntimeError(
                f"paged KV block id exceeds cache capacity: block_id={block_id}, num_blocks={cache.shape[0]}"
            )
        take = min(page_size, remaining)
        pieces.append(cache[block_id, :take])
        remaining -= take
    if remaining != 0 or not pieces:
        raise RuntimeError(f"invalid block table for paged KV reference: context_len={context_len}, remaining={remaining}")
    return torch.cat(pieces, dim=0)


def decode_reference_qdtype(q, k_cache, v_cache, block_tables, context_lens, scale, *,
                            k_scale_cache=None, v_scale_cache=None) -> torch.Tensor:
    """``paged_decode_attention_reference`` (ops/paged_attention_reference.py:249-320).

    The reference CPU path: per sequence gather pages until ``context_len``,
    dequantize in ``q.dtype`` (bf16 product rounding), expand GQA with
    ``repeat_interleave`` (:125-145) and run SDPA in ``q.dtype``.
    """

    batch, num_heads, head_dim = q.shape
    num_kv_heads = k_cache.shape[2]
    groups = num_heads // num_kv_heads
    outputs = []
    for b in range(batch):
        ctx = int(context_lens[b].item())
        keys = _gather_sequence(k_cache, block_tables[b], ctx)
        values = _gather_sequence(v_cache, block_tables[b], ctx)
        ks = vs = None
        if k_scale_cache is not None:
            ks = _gather_sequence(k_scale_cache, block_tables[b], ctx)
            vs = _gather_sequence(v_scale_cache, block_tables[b], ctx)
        keys = dequantize(keys, ks, q.dtype)
        values = dequantize(values, vs, q.dtype)
        if groups != 1:
            keys = keys.repeat_interleave(groups, dim=1)
            values = values.repeat_interleave(groups, dim=1)
        query = q[b].unsqueeze(0).unsqueeze(2)
        output = F.scaled_dot_product_attention(
            query, keys.transpose(0, 1).unsqueeze(0), values.transpose(0, 1).unsqueeze(0),
            is_causal=False, scale=scale,
        )
        outputs.append(output.squeeze(0).squeeze(1))
    return torch.stack(outputs, dim=0)


def decode_reference_fp32(q, k_payload, v_payload, k_scales, v_scales, block_tables, context_lens,
                          scale) -> torch.Tensor:
    """The reference's independent test oracle (tests/test_scaled_fp8_kv_cache.py:71-102).

    fp32 dequantization of whole blocks, ``[:context_len]`` slicing, fp32 SDPA,
    result cast to ``q.dtype``.  Block ids are used as given (all must be valid).
    """

    k_cache = k_payload.float()
    v_cache = v_payload.float()
    if k_scales is not None:
        k_cache = k_cache * k_scales.float().unsqueeze(-1)
        v_cache = v_cache * v_scales.float().unsqueeze(-1)
    num_heads = q.shape[1]
    num_kv_heads = k_payload.shape[2]
    groups = num_heads // num_kv_heads
    outputs = []
    for row in range(q.shape[0]):
        ctx = int(context_lens[row].item())
        block_ids = block_tables[row].long()
        keys = k_cache[block_ids].reshape(-1, num_kv_heads, q.shape[-1])[:ctx]
        values = v_cache[block_ids].reshape(-1, num_kv_heads, q.shape[-1])[:ctx]
        keys = keys.repeat_interleave(groups, dim=1)
        values = values.repeat_interleave(groups, dim=1)
        output = F.scaled_dot_product_attention(
            q[row].float().view(1, num_heads, 1, q.shape[-1]),
            keys.transpose(0, 1).unsqueeze(0), values.transpose(0, 1).unsqueeze(0),
            is_causal=False, scale=scale,
        )
        outputs.append(output.squeeze(0).squeeze(1))
    return torch.stack(outputs).to(q.dtype)


def decode_bruteforce_f64(q, keys, values, scale) -> torch.Tensor:
    """Textbook attention for ONE sequence in float64 with explicit loops.

    ``q``: [Hq, D]; ``keys``/``values``: [n, Hkv, D] already dequantized.
    Used only to pin the other formulations on tiny shapes.
    """

    num_heads, head_dim = q.shape
    n, num_kv_heads, _ = keys.shape
    groups = num_heads // num_kv_heads
    out = torch.zeros(num_heads, head_dim, dtype=torch.float64)
    for h in range(num_heads):
        kh = h // groups
        logits = [float(sum(float(q[h, d]) * float(keys[t, kh, d]) for d in range(head_dim))) * scale
                  for t in range(n)]
        if not logits:
            continue
        m = max(logits)
        weights = [math.exp(x - m) for x in logits]
        total = sum(weights)
        for d in range(head_dim):
            out[h, d] = sum(w * float(values[t, kh, d]) for t, w in enumerate(weights)) / total
    return out


# --------------------------------------------------------------------------- prefill


def _prefill_lengths(cu_seqlens_q, context_lens, i: int) -> tuple[int, int, int]:
    query_start = int(cu_seqlens_q[i])
    query_len = int(cu_seqlens_q[i + 1]) - query_start
    context_len = int(context_lens[i])
    if query_len <= 0 or context_len < query_len:
        raise RuntimeError(f"invalid paged prefill lengths: query={query_len} context={context_len}")
    return query_start, query_len, context_len


def prefill_reference_qdtype(q, k_cache, v_cache, block_tables, context_lens, cu_seqlens_q, *, num_heads,
                             num_kv_heads, scale, k_scale_cache=None, v_scale_cache=None) -> torch.Tensor:
    """``paged_prefill_attention_reference`` (ops/paged_attention_reference.py:185-246).

    Per sequence i: query rows ``cu[i]:cu[i+1]``; ``prefix = context_len -
    query_len``; gather the pages up to ``context_len`` (:22-63), dequantize
    in ``q.dtype`` (:102-122), expand GQA (:125-145), and run SDPA with the
    causal mask ``key_pos <= prefix + j`` (:228-240).  Outputs are
    concatenated in sequence order.
    """

    outputs = []
    groups = num_heads // num_kv_heads
    for i in range(context_lens.numel()):
        start, query_len, context_len = _prefill_lengths(cu_seqlens_q, context_lens, i)
        prefix = context_len - query_len
        keys = _gather_sequence(k_cache, block_tables[i], context_len)
        values = _gather_sequence(v_cache, block_tables[i], context_len)
        ks = vs = None
        if k_scale_cache is not None:
            ks = _gather_sequence(k_scale_cache, block_tables[i], context_len)
            vs = _gather_sequence(v_scale_cache, block_tables[i], context_len)
        keys = dequantize(keys, ks, q.dtype)
        values = dequantize(values, vs, q.dtype)
        if groups != 1:
            keys = keys.repeat_interleave(groups, dim=1)
            values = values.repeat_interleave(groups, dim=1)
        queries = q[start:start + query_len].transpose(0, 1).unsqueeze(0)
        mask = (torch.arange(context_len).unsqueeze(0) <= torch.arange(prefix, context_len).unsqueeze(1))
        output = F.scaled_dot_product_attention(
            queries, keys.transpose(0, 1).unsqueeze(0), values.transpose(0, 1).unsqueeze(0),
            attn_mask=mask.unsqueeze(0).unsqueeze(0), is_causal=False, scale=scale,
        )
        outputs.append(output.squeeze(0).transpose(0, 1))
    return torch.cat(outputs, dim=0)


def prefill_reference_fp32(q, k_cache, v_cache, block_tables, context_lens, cu_seqlens_q, *, num_heads,
                           num_kv_heads, scale, k_scale_cache=None, v_scale_cache=None,
                           compute_dtype=torch.float64) -> torch.Tensor:
    """The same attention with fp32 dequantization (``fp8 -> fp32 * scale``, as
    the reference's decode test oracle dequantizes, tests/test_scaled_fp8_kv_cache.py:71-102)
    and the softmax evaluated in ``compute_dtype`` (float64 by default): the
    exact causal attention of the dequantized cache.  Result in ``q.dtype``.
    """

    outputs = []
    groups = num_heads // num_kv_heads
    for i in range(context_lens.numel()):
        start, query_len, context_len = _prefill_lengths(cu_seqlens_q, context_lens, i)
        prefix = context_len - query_len
        keys = _gather_sequence(k_cache, block_tables[i], context_len).to(torch.float32)
        values = _gather_sequence(v_cache, block_tables[i], context_len).to(torch.float32)
        if k_scale_cache is not None:
            keys = keys * _gather_sequence(k_scale_cache, block_tables[i], context_len).float().unsqueeze(-1)
            values = values * _gather_sequence(v_scale_cache, block_tables[i], context_len).float().unsqueeze(-1)
        keys = keys.to(compute_dtype).repeat_interleave(groups, dim=1)        # [ctx, Hq, D]
        values = values.to(compute_dtype).repeat_interleave(groups, dim=1)
        queries = q[start:start + query_len].to(compute_dtype)               # [n, Hq, D]
        scores = torch.einsum("nhd,khd->hnk", queries, keys) * scale
        visible = torch.arange(context_len).unsqueeze(0) <= torch.arange(prefix, context_len).unsqueeze(1)
        scores = scores.masked_fill(~visible.unsqueeze(0), float("-inf"))
        probs = torch.softmax(scores, dim=-1)
        outputs.append(torch.einsum("hnk,khd->nhd", probs, values))
    return torch.cat(outputs, dim=0).to(q.dtype)


def prefill_bruteforce_f64(queries, keys, values, prefix: int, scale: float) -> torch.Tensor:
    """Causal attention of ONE sequence in float64 with explicit loops.

    ``queries``: [n, Hq, D]; ``keys``/``values``: [prefix + n, Hkv, D] already
    dequantized; query j attends to keys ``0 .. prefix + j``.
    """

    n, num_heads, head_dim = queries.shape
    groups = num_heads // keys.shape[1]
    out = torch.zeros(n, num_heads, head_dim, dtype=torch.float64)
    for j in range(n):
        for h in range(num_heads):
            kh = h // groups
            logits = [sum(float(queries[j, h, d]) * float(keys[t, kh, d]) for d in range(head_dim)) * scale
                      for t in range(prefix + j + 1)]
            m = max(logits)
            weights = [math.exp(x - m) for x in logits]
            total = sum(weights)
            for d in range(head_dim):
                out[j, h, d] = sum(w * float(values[t, kh, d]) for t, w in enumerate(weights)) / total
    return out


if os.environ.get("PRISM_ORACLE_BUILD_ON_IMPORT"):
    build_oracle()
