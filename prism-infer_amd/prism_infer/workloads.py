"""Seeded synthetic inputs for the scaled-FP8 paged KV path.

Shapes follow the five measured configurations of the KV path (all 32 query
heads over 8 KV heads, head_dim 128, 256-token pages unless stated):

* ``decode_single``   -- B=1, one 2048-token context in 8 pages placed at a
                         seeded permutation of a 64-page pool.
* ``store_prefill``   -- 8192 bf16 K/V tokens ~N(0,1) with 1% outliers x20,
                         scattered by a seeded slot permutation into 512 pages.
* ``decode_qwen_vl``  -- B=1, 1800 tokens (8 x 196 visual + 232 text) in 8
                         pages of a 64-page pool.
* ``decode_mixed``    -- B=64, lengths ~U{1024..16384}; the 32 longest share
                         one 4096-token prefix (16 physical pages); every
                         other token sits in private pages drawn without
                         replacement from an 8192-page pool; W = 64.
* ``compaction``      -- 64 prefixes x 8192 tokens, seeded keep-mask dropping
                         ~30% of visual positions [64, 8192), >= 768 kept.
* ``decode_long``     -- B=256, 32k context each, pages scattered in a pool.
* ``prefill_chunked`` -- paged prefill: B=4 sequences, each an 8192-token
                         cached prefix plus a 2048-token chunk (already
                         stored), 40 pages per sequence drawn without
                         replacement from a 512-page pool.

Index metadata is drawn on the CPU with ``torch.Generator`` so it is identical
on every machine.  K/V values are drawn as bf16 N(0,1) on the target device
(seeded) and quantised with the library's own scaled store; tests compare the
resulting pages against the CPU oracle separately.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

NUM_HEADS = 32
NUM_KV_HEADS = 8
HEAD_DIM = 128
PAGE_SIZE = 256
FP8 = torch.float8_e4m3fn


@dataclass
class DecodeWorkload:
    name: str
    q: torch.Tensor
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    k_scale: torch.Tensor
    v_scale: torch.Tensor
    block_tables: torch.Tensor
    context_lens: torch.Tensor
    max_context_len: torch.Tensor
    scale: float
    used_pages: torch.Tensor            # unique physical pages referenced (CPU int64)
    shared_prefix_pages: int = 0
    meta: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return self.q.shape[0]

    def unique_kv_tokens(self) -> int:
        """Distinct (page, row) KV entries read: shared prefix rows count once."""

        return int(self.meta["unique_tokens"])

    def algorithmic_bytes(self) -> int:
        """Unique bytes a decode pass must move (see the measurement contract)."""

        kv_heads, dim = self.k_cache.shape[2], self.k_cache.shape[3]
        per_token = 2 * kv_heads * dim + 2 * kv_heads * 4
        q_out = 2 * self.q.numel() * self.q.element_size()
        tables = self.batch * self.block_tables.shape[1] * 4
        return self.unique_kv_tokens() * per_token + q_out + tables + self.batch * 4


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def fill_pages(k_cache, v_cache, k_scale, v_scale, pages: torch.Tensor, seed: int, *, chunk_pages: int = 512) -> None:
    """Fill ``pages`` of the caches with quantised bf16 N(0,1) K/V (device-side, seeded)."""

    from prism_infer.ops.kv_cache_store import store_kvcache  # noqa: PLC0415

    device = k_cache.device
    _, page_size, kv_heads, dim = k_cache.shape
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    pages = pages.to(torch.int64)
    for start in range(0, pages.numel(), chunk_pages):
        chunk = pages[start:start + chunk_pages].to(device)
        tokens = chunk.numel() * page_size
        key = torch.randn(tokens, kv_heads, dim, generator=gen, device=device, dtype=torch.bfloat16)
        value = torch.randn(tokens, kv_heads, dim, generator=gen, device=device, dtype=torch.bfloat16)
        slots = (chunk[:, None] * page_size + torch.arange(page_size, device=device)[None, :]).reshape(-1)
        store_kvcache(key, value, k_cache, v_cache, slots.to(torch.int32), k_scale, v_scale)


def _alloc_pool(num_pages: int, device, *, page_size=PAGE_SIZE, kv_heads=NUM_KV_HEADS, dim=HEAD_DIM):
    k = torch.empty(num_pages, page_size, kv_heads, dim, dtype=FP8, device=device)
    v = torch.empty_like(k)
    ks = torch.empty(num_pages, page_size, kv_heads, dtype=torch.float32, device=device)
    vs = torch.empty_like(ks)
    return k, v, ks, vs


def _finish(name, q, pool, tables, lens, seed, used, unique_tokens, shared=0, meta=None, fill=True):
    k, v, ks, vs = pool
    if fill:
        fill_pages(k, v, ks, vs, used, seed + 1)
    device = k.device
    lens_t = torch.tensor(lens, dtype=torch.int32)
    m = dict(meta or {})
    m["unique_tokens"] = unique_tokens
    return DecodeWorkload(
        name=name,
        q=q,
        k_cache=k, v_cache=v, k_scale=ks, v_scale=vs,
        block_tables=tables.to(device),
        context_lens=lens_t.to(device),
        max_context_len=lens_t.max().reshape(1).to(device),
        scale=HEAD_DIM ** -0.5,
        used_pages=used,
        shared_prefix_pages=shared,
        meta=m,
    )


def decode_single(device, seed: int = 20260801, *, context_len: int = 2048, pool_pages: int = 64,
                  name: str = "decode_single", fill: bool = True) -> DecodeWorkload:
    g = _gen(seed)
    pages_needed = math.ceil(context_len / PAGE_SIZE)
    perm = torch.randperm(pool_pages, generator=g)[:pages_needed]
    q = torch.randn(1, NUM_HEADS, HEAD_DIM, generator=g, dtype=torch.bfloat16).to(device)
    tables = perm.to(torch.int32).reshape(1, -1)
    pool = _alloc_pool(pool_pages, device)
    return _finish(name, q, pool, tables, [context_len], seed, perm.clone(), context_len, fill=fill)


def decode_qwen_vl(device, seed: int = 20260803, *, fill: bool = True) -> DecodeWorkload:
    ctx = 8 * 196 + 232
    return decode_single(device, seed, context_len=ctx, name="decode_qwen_vl", fill=fill)


def decode_mixed(device, seed: int = 20260804, *, batch: int = 64, min_len: int = 1024, max_len: int = 16384,
                 shared_seqs: int = 32, prefix_tokens: int = 4096, pool_pages: int = 8192,
                 fill: bool = True) -> DecodeWorkload:
    g = _gen(seed)
    lens = torch.randint(min_len, max_len + 1, (batch,), generator=g)
    order = torch.argsort(lens, descending=True, stable=True)
    sharing = set(order[:shared_seqs].tolist())
    for b in sharing:
        if int(lens[b]) <= prefix_tokens:
            raise RuntimeError("a prefix-sharing sequence must be longer than the shared prefix")
    width = math.ceil(max_len / PAGE_SIZE)
    prefix_pages = prefix_tokens // PAGE_SIZE
    perm = torch.randperm(pool_pages, generator=g)
    shared_pages = perm[:prefix_pages]
    cursor = prefix_pages
    tables = torch.full((batch, width), -1, dtype=torch.int32)
    unique = prefix_tokens if sharing else 0
    for b in range(batch):
        n = int(lens[b])
        if b in sharing:
            private = math.ceil((n - prefix_tokens) / PAGE_SIZE)
            row = torch.cat([shared_pages, perm[cursor:cursor + private]])
            unique += n - prefix_tokens
        else:
            private = math.ceil(n / PAGE_SIZE)
            row = perm[cursor:cursor + private]
            unique += n
        cursor += private
        tables[b, : row.numel()] = row.to(torch.int32)
    if cursor > pool_pages:
        raise RuntimeError("pool too small for the sampled lengths")
    used = perm[:cursor].clone()
    q = torch.randn(batch, NUM_HEADS, HEAD_DIM, generator=g, dtype=torch.bfloat16).to(device)
    pool = _alloc_pool(pool_pages, device)
    return _finish("decode_mixed", q, pool, tables, lens.tolist(), seed, used, unique,
                   shared=prefix_pages, meta={"sharing": sorted(sharing)}, fill=fill)


def decode_long(device, seed: int = 20260805, *, batch: int = 256, context_len: int = 32768,
                pool_pages: int | None = None, fill: bool = True) -> DecodeWorkload:
    g = _gen(seed)
    pages_per = math.ceil(context_len / PAGE_SIZE)
    pool_pages = pool_pages or batch * pages_per
    perm = torch.randperm(pool_pages, generator=g)[: batch * pages_per]
    tables = perm.to(torch.int32).reshape(batch, pages_per)
    q = torch.randn(batch, NUM_HEADS, HEAD_DIM, generator=g, dtype=torch.bfloat16).to(device)
    pool = _alloc_pool(pool_pages, device)
    return _finish("decode_long", q, pool, tables, [context_len] * batch, seed, perm.clone(),
                   batch * context_len, fill=fill)


def fill_slots(k_cache, v_cache, k_scale, v_scale, slots: torch.Tensor, seed: int, *, chunk: int = 1 << 17) -> None:
    """Fill individual slots (flat ``block * P + offset``) with quantised bf16 N(0,1) K/V."""

    from prism_infer.ops.kv_cache_store import store_kvcache  # noqa: PLC0415

    device = k_cache.device
    _, _, kv_heads, dim = k_cache.shape
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    slots = slots.to(device=device, dtype=torch.int32)
    for start in range(0, slots.numel(), chunk):
        sl = slots[start:start + chunk]
        key = torch.randn(sl.numel(), kv_heads, dim, generator=gen, device=device, dtype=torch.bfloat16)
        value = torch.randn(sl.numel(), kv_heads, dim, generator=gen, device=device, dtype=torch.bfloat16)
        store_kvcache(key, value, k_cache, v_cache, sl, k_scale, v_scale)


def decode_long_compacted(device, seed: int = 20260805, *, batch: int = 256, context_len: int = 32768,
                          compacted: int = 64, pool_pages: int | None = None) -> DecodeWorkload:
    """Config 5 as one chain: compaction, then long-context decode over its output.

    The 64 prefixes of :func:`compaction_plans` (8192 tokens each, ~30 % of
    the visual positions dropped) are written into their source pages, then
    moved with ``compact_kv_slots`` (payload and scales of K and V) into new
    dense destination pages.  Sequences ``0 .. compacted - 1`` of the decode
    batch start with those destination pages: their first ``kept`` tokens are
    the compacted prefix and the following ``context_len - kept`` tokens fill
    the rest of the last destination page and private pages, as later tokens
    of a compacted sequence do (kv_compaction_coordinator.py:86-98; the block
    table keeps the compacted prefix and grows after it).  The other
    sequences hold ``context_len`` tokens in private pages.  Pages are
    scattered over a pool of ``pool_pages`` pages.  ``meta`` carries the
    compaction plans and slot tensors for checking.
    """

    from prism_infer.ops.kv_compaction import compact_kv_slots  # noqa: PLC0415

    pages_per = math.ceil(context_len / PAGE_SIZE)
    cw_need = compacted * (8192 // PAGE_SIZE) * 2
    need = cw_need + batch * pages_per
    pool_pages = pool_pages or need
    if pool_pages < need:
        raise RuntimeError(f"pool of {pool_pages} pages is smaller than the {need} the chain needs")
    cw = compaction_plans(prefixes=compacted, pool_pages=pool_pages)
    g = _gen(seed)
    taken = set()
    for plan in cw.plans:
        taken.update(plan.old_block_table)
        taken.update(plan.new_block_table)
    free = [p for p in torch.randperm(pool_pages, generator=g).tolist() if p not in taken]
    k, v, ks, vs = _alloc_pool(pool_pages, device)
    # 1. the prefixes' K/V in their source pages, then the compaction
    src_pages = torch.tensor(sorted({p for plan in cw.plans for p in plan.old_block_table}), dtype=torch.int64)
    fill_pages(k, v, ks, vs, src_pages, seed + 2)
    src = torch.tensor([x for plan in cw.plans for x in plan.source_slots], dtype=torch.long, device=device)
    dst = torch.tensor([x for plan in cw.plans for x in plan.destination_slots], dtype=torch.long, device=device)
    n_slots = pool_pages * PAGE_SIZE
    compact_kv_slots(k.view(1, 1, n_slots, NUM_KV_HEADS, HEAD_DIM), src, dst)
    compact_kv_slots(v.view(1, 1, n_slots, NUM_KV_HEADS, HEAD_DIM), src, dst)
    compact_kv_slots(ks.view(1, 1, n_slots, NUM_KV_HEADS), src, dst)
    compact_kv_slots(vs.view(1, 1, n_slots, NUM_KV_HEADS), src, dst)
    # 2. block tables: compacted prefix pages, then private pages
    tables = torch.full((batch, pages_per), -1, dtype=torch.int32)
    cursor = 0
    tail_slots = []
    private_pages = []
    for b in range(batch):
        if b < compacted:
            plan = cw.plans[b]
            kept = plan.physical_prompt_len
            head = list(plan.new_block_table)
            used_in_last = kept - (len(head) - 1) * PAGE_SIZE
            last = head[-1]
            tail_slots.extend(last * PAGE_SIZE + o for o in range(used_in_last, PAGE_SIZE))
            rest = max(0, math.ceil((context_len - len(head) * PAGE_SIZE) / PAGE_SIZE))
            row = head + free[cursor:cursor + rest]
        else:
            rest = pages_per
            row = free[cursor:cursor + rest]
        private_pages.extend(free[cursor:cursor + rest])
        cursor += rest
        tables[b, :len(row)] = torch.tensor(row, dtype=torch.int32)
    if cursor > len(free):
        raise RuntimeError("pool too small for the decode batch")
    # 3. the tokens after each compacted prefix, and every private page
    fill_slots(k, v, ks, vs, torch.tensor(tail_slots, dtype=torch.int64), seed + 3)
    fill_pages(k, v, ks, vs, torch.tensor(private_pages, dtype=torch.int64), seed + 1)
    q = torch.randn(batch, NUM_HEADS, HEAD_DIM, generator=g, dtype=torch.bfloat16).to(device)
    used = torch.unique(tables[tables >= 0].to(torch.int64))
    meta = {"compaction": cw, "compaction_src": src, "compaction_dst": dst, "compacted": compacted}
    return _finish("decode_long_compacted", q, (k, v, ks, vs), tables, [context_len] * batch, seed, used,
                   batch * context_len, meta=meta, fill=False)


@dataclass
class PrefillWorkload:
    q: torch.Tensor                     # [total_q, Hq, D] bf16
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    k_scale: torch.Tensor
    v_scale: torch.Tensor
    block_tables: torch.Tensor          # int32 [B, W]
    context_lens: torch.Tensor          # int32 [B]
    cu_seqlens_q: torch.Tensor          # int32 [B + 1]
    scale: float
    query_lens: list
    ctx_lens: list

    @property
    def num_heads(self) -> int:
        return self.q.shape[1]

    @property
    def num_kv_heads(self) -> int:
        return self.k_cache.shape[2]

    def attended_pairs(self) -> int:
        """Sum over sequences of (query, key) pairs the causal mask admits."""

        total = 0
        for n, ctx in zip(self.query_lens, self.ctx_lens):
            prefix = ctx - n
            total += n * prefix + n * (n + 1) // 2
        return total

    def flops(self) -> int:
        """2 * D multiply-adds per (query head, visible key) for QK^T and again for PV."""

        return 4 * self.q.shape[2] * self.num_heads * self.attended_pairs()

    def algorithmic_bytes(self) -> int:
        kv_heads, dim = self.k_cache.shape[2], self.k_cache.shape[3]
        per_token = 2 * kv_heads * dim + 2 * kv_heads * 4
        q_out = 2 * self.q.numel() * self.q.element_size()
        meta = self.block_tables.numel() * 4 + len(self.ctx_lens) * 8 + 4
        return sum(self.ctx_lens) * per_token + q_out + meta


def prefill_chunked(device, seed: int = 20260807, *, batch: int = 4, prefix: int = 8192, chunk: int = 2048,
                    pool_pages: int = 512, fill: bool = True) -> PrefillWorkload:
    g = _gen(seed)
    ctx = prefix + chunk
    pages_per = math.ceil(ctx / PAGE_SIZE)
    if batch * pages_per > pool_pages:
        raise ValueError("pool too small for the prefill workload")
    perm = torch.randperm(pool_pages, generator=g)[:batch * pages_per].view(batch, pages_per)
    q = torch.randn(batch * chunk, NUM_HEADS, HEAD_DIM, generator=g, dtype=torch.float32).to(torch.bfloat16)
    pool = _alloc_pool(pool_pages, device)
    if fill:
        fill_pages(*pool, perm.reshape(-1), seed + 1)
    cu = torch.arange(batch + 1, dtype=torch.int32) * chunk
    return PrefillWorkload(
        q=q.to(device), k_cache=pool[0], v_cache=pool[1], k_scale=pool[2], v_scale=pool[3],
        block_tables=perm.to(torch.int32).to(device),
        context_lens=torch.full((batch,), ctx, dtype=torch.int32).to(device),
        cu_seqlens_q=cu.to(device), scale=HEAD_DIM ** -0.5,
        query_lens=[chunk] * batch, ctx_lens=[ctx] * batch,
    )


@dataclass
class StoreWorkload:
    key: torch.Tensor
    value: torch.Tensor
    slot_mapping: torch.Tensor
    num_pages: int

    def algorithmic_bytes(self) -> int:
        t, h, d = self.key.shape
        return 2 * t * h * d * self.key.element_size() + 2 * t * h * d + 2 * t * h * 4 + t * 4


def store_prefill(device, seed: int = 20260802, *, tokens: int = 8192, num_pages: int = 512,
                  outlier_rate: float = 0.01, outlier_scale: float = 20.0) -> StoreWorkload:
    g = _gen(seed)
    shape = (tokens, NUM_KV_HEADS, HEAD_DIM)
    key = torch.randn(shape, generator=g, dtype=torch.float32)
    value = torch.randn(shape, generator=g, dtype=torch.float32)
    for t in (key, value):
        mask = torch.rand(shape, generator=g) < outlier_rate
        t[mask] *= outlier_scale
    slots = torch.randperm(num_pages * PAGE_SIZE, generator=g)[:tokens].to(torch.int32)
    return StoreWorkload(key.to(torch.bfloat16).to(device), value.to(torch.bfloat16).to(device),
                         slots.to(device), num_pages)


@dataclass
class CompactionWorkload:
    plans: list            # CompactionSlots per prefix
    num_pages: int
    kept: int

    def algorithmic_bytes(self, layers: int = 1, kv_heads: int = NUM_KV_HEADS, dim: int = HEAD_DIM) -> int:
        per_token = 2 * kv_heads * dim + 2 * kv_heads * 4
        return 2 * self.kept * per_token * layers + 16 * self.kept


def compaction_plans(seed: int = 20260806, *, prefixes: int = 64, prefix_tokens: int = 8192,
                     text_tokens: int = 64, drop: float = 0.3, min_keep: int = 768,
                     in_place: bool = False, pool_pages: int | None = None) -> CompactionWorkload:
    from prism_infer.engine.kv_compaction_plan import plan_in_place, plan_out_of_place  # noqa: PLC0415

    g = _gen(seed)
    pages_per = prefix_tokens // PAGE_SIZE
    need = prefixes * pages_per * (1 if in_place else 2)
    pool_pages = pool_pages or need
    perm = torch.randperm(pool_pages, generator=g)
    plans = []
    kept_total = 0
    for p in range(prefixes):
        old = perm[p * pages_per:(p + 1) * pages_per].tolist()
        drop_mask = torch.rand(prefix_tokens - text_tokens, generator=g) < drop
        keep = torch.cat([torch.ones(text_tokens, dtype=torch.bool), ~drop_mask])
        positions = torch.nonzero(keep).flatten().tolist()
        if len(positions) < min_keep:
            raise RuntimeError("keep-mask kept fewer tokens than the configured minimum")
        if in_place:
            plan = plan_in_place(old, positions, PAGE_SIZE, logical_prompt_len=prefix_tokens)
        else:
            base = prefixes * pages_per + p * pages_per
            dest = perm[base:base + pages_per].tolist()
            plan = plan_out_of_place(old, positions, PAGE_SIZE, dest)
        plans.append(plan)
        kept_total += plan.physical_prompt_len
    return CompactionWorkload(plans, pool_pages, kept_total)


__all__ = [
    "CompactionWorkload",
    "DecodeWorkload",
    "StoreWorkload",
    "compaction_plans",
    "decode_long",
    "decode_long_compacted",
    "decode_mixed",
    "decode_qwen_vl",
    "decode_single",
    "fill_pages",
    "fill_slots",
    "store_prefill",
]
