"""Benchmark of the scaled-FP8 paged KV hot path on one MI355X.

Headline: paged-decode achieved HBM GB/s (and % of the 8 TB/s peak) plus
us/layer on the batch-64 mixed-context workload (``decode_mixed``: 64
sequences, lengths U[1k, 16k], 32 of them sharing one 4096-token prefix,
32 q / 8 kv heads, head_dim 128, 256-token scaled-FP8 pages).  A step is one
layer's decode over the batch (plan check, streaming kernel, merge).  Steps rotate over ``--layers`` independent KV pools so that each
step reads its pages cold from HBM (the 256 MB MALL cannot hold a layer).

``value`` = algorithmic bytes / time per step, where algorithmic bytes count
every distinct (page, used row) once (2112 B per token per layer for K+V
payload and scales; shared-prefix rows once) plus q, out, block tables and
context lengths.  ``roofline.achieved`` uses the same bytes over the split-K
kernel's own average duration, measured with HIP events on the stream it is
launched on.  ``cpu_baseline`` times the CPU restatement of the reference's
decode path (per-sequence page gather, bf16 dequant, GQA expand, SDPA) on a
bounded sample of the same workload's sequences.

    python bench.py [--gpus 1] [--steps 50] [--warmup 100]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO_ROOT = Path(__file__).resolve().parent
for _p in (REPO_ROOT, REPO_ROOT / "prism-infer_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "paged-decode achieved HBM GB/s (% of peak) + µs/layer, batch 64 mixed ctx"
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK = 2.5e15  # dense bf16/fp16 MFMA, FLOP/s
TRAFFIC_FILE = REPO_ROOT / "profiles" / "decode_mixed_traffic.json"
# config 5's decode pool: ~120 GB of scaled-FP8 pages (256 x 128 of them are used)
LONG_POOL_PAGES = 221_946


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _time_loop(fn, steps: int, torch) -> float:
    """Seconds per call of ``fn`` over ``steps`` calls, HIP events on the current stream."""

    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(steps):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / steps


def _time_queued(fn, calls: int, torch, *, reps: int = 5, flush=None) -> float:
    """Median GPU seconds per call of ``fn`` launched eagerly behind a GPU spin.

    Each repetition runs ``flush()``, then a spin kernel long enough for the
    host to enqueue all ``calls`` calls before the start event is reached, so
    the timed span is the calls' own GPU time back to back (no host launch
    overhead and no graph-launch latency).  If the start event has already
    completed when the host finishes enqueueing, the spin was too short: it
    is doubled and the repetition is repeated."""

    for i in range(calls):  # warm-up (allocations, plans)
        fn(i)
    torch.cuda.synchronize()
    spin = 2_000_000 + calls * 200_000
    times = []
    while len(times) < reps:
        if flush is not None:
            flush()
        torch.cuda._sleep(spin)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(calls):
            fn(i)
        end.record()
        late = start.query()
        torch.cuda.synchronize()
        if late:
            spin *= 2
            if spin > 1 << 32:
                raise RuntimeError("host cannot enqueue the timed calls ahead of the GPU")
            continue
        times.append(start.elapsed_time(end) / 1e3 / calls)
    times.sort()
    return times[len(times) // 2]


def _cpu_decode_sample(w, budget_s: float, torch) -> dict:
    """The CPU restatement of the reference decode path (paged_attention_reference.py:249-320)
    over the first sequences of a decode workload, until ``budget_s`` of CPU time."""

    import oracle  # noqa: PLC0415  (checker/baseline only)

    tables = w.block_tables.cpu()
    lens = w.context_lens.cpu()
    done_bytes = 0
    seqs = 0
    elapsed = 0.0
    per_token = 2 * 8 * 128 + 2 * 8 * 4
    for b in range(w.batch):
        n = int(lens[b])
        pages = tables[b][: (n + 255) // 256].long()
        idx = pages.to(w.k_cache.device)
        k = w.k_cache.view(torch.uint8).index_select(0, idx).cpu().view(torch.float8_e4m3fn)
        v = w.v_cache.view(torch.uint8).index_select(0, idx).cpu().view(torch.float8_e4m3fn)
        ks = w.k_scale.index_select(0, idx).cpu()
        vs = w.v_scale.index_select(0, idx).cpu()
        local = torch.arange(pages.numel(), dtype=torch.int32).reshape(1, -1)
        q = w.q[b:b + 1].cpu()
        t0 = time.perf_counter()
        oracle.decode_reference_qdtype(q, k, v, local, lens[b:b + 1], w.scale, k_scale_cache=ks, v_scale_cache=vs)
        elapsed += time.perf_counter() - t0
        done_bytes += n * per_token + 2 * q.numel() * 2 + local.numel() * 4 + 4
        seqs += 1
        if elapsed >= budget_s:
            break
    return {"GBps": round(done_bytes / elapsed / 1e9, 4), "seconds": round(elapsed, 2), "sequences": seqs,
            "us_per_layer_equiv": round(elapsed / seqs * w.batch * 1e6, 1)}


def _cpu_config1(dev, budget_s: float, torch, workloads) -> dict:
    """Config 1 as the reference runs it on the CPU: B = 1, 2048 tokens in 8
    pages of a 64-page pool, decode_reference_qdtype repeated for ``budget_s``."""

    import oracle  # noqa: PLC0415

    w = workloads.decode_single(dev)
    q = w.q.cpu()
    k = w.k_cache.view(torch.uint8).cpu().view(torch.float8_e4m3fn)
    v = w.v_cache.view(torch.uint8).cpu().view(torch.float8_e4m3fn)
    ks, vs = w.k_scale.cpu(), w.v_scale.cpu()
    tables, lens = w.block_tables.cpu(), w.context_lens.cpu()
    reps, elapsed = 0, 0.0
    while elapsed < budget_s or reps < 3:
        t0 = time.perf_counter()
        oracle.decode_reference_qdtype(q, k, v, tables, lens, w.scale, k_scale_cache=ks, v_scale_cache=vs)
        elapsed += time.perf_counter() - t0
        reps += 1
    s = elapsed / reps
    return {"us_per_layer": round(s * 1e6, 1), "GBps": round(w.algorithmic_bytes() / s / 1e9, 4), "reps": reps,
            "sample": "config 1 in full (B=1, 2048 tokens), reference CPU path (page gather, bf16 dequant, GQA "
                      "expand, SDPA)"}


def _cpu_store(dev, budget_s: float, torch, workloads) -> dict:
    """Config 2's store as the reference's CPU path runs it (a per-token torch loop,
    kv_cache_store.py:170-230) over the first tokens of the 8192-token chunk until
    ``budget_s``; the whole chunk's time is extrapolated from the tokens done."""

    import oracle  # noqa: PLC0415

    sw = workloads.store_prefill(dev)
    key, value, slots = sw.key.cpu(), sw.value.cpu(), sw.slot_mapping.cpu()
    kc = torch.zeros(sw.num_pages, 256, 8, 128, dtype=torch.uint8).view(torch.float8_e4m3fn)
    vc = torch.zeros_like(kc.view(torch.uint8)).view(torch.float8_e4m3fn)
    ksc = torch.zeros(sw.num_pages, 256, 8)
    vsc = torch.zeros_like(ksc)
    done, elapsed, chunk = 0, 0.0, 256
    while done < key.shape[0] and elapsed < budget_s:
        sl = slice(done, done + chunk)
        t0 = time.perf_counter()
        oracle.store_scaled_torch_loop(key[sl], value[sl], kc, vc, slots[sl], ksc, vsc)
        elapsed += time.perf_counter() - t0
        done += key[sl].shape[0]
    per_token = sw.algorithmic_bytes() / key.shape[0]
    return {"us_chunk_equiv": round(elapsed / done * key.shape[0] * 1e6, 1),
            "GBps": round(done * per_token / elapsed / 1e9, 5), "tokens": done,
            "sample": f"first {done} of {key.shape[0]} tokens of config 2, reference CPU path (per-token loop)"}


def _cpu_compaction(budget_s: float, torch, workloads) -> dict:
    """Config 5's compaction as the reference's CPU path runs it
    (index_select + index_copy_, kv_compaction.py:111-112) on payload and scale
    caches at L = 1 (payload moved as bytes), whole plan, one call each."""

    cw = workloads.compaction_plans()
    slots = cw.num_pages * 256
    src = torch.tensor([x for p in cw.plans for x in p.source_slots], dtype=torch.long)
    dst = torch.tensor([x for p in cw.plans for x in p.destination_slots], dtype=torch.long)
    payload = torch.zeros(2, 1, slots, 8, 128, dtype=torch.uint8)
    scales = torch.zeros(2, 1, slots, 8, dtype=torch.float32)
    import oracle  # noqa: PLC0415

    reps, elapsed = 0, 0.0
    while elapsed < budget_s or reps < 1:
        t0 = time.perf_counter()
        oracle.compact_slots_torch(payload, src, dst)
        oracle.compact_slots_torch(scales, src, dst)
        elapsed += time.perf_counter() - t0
        reps += 1
    s = elapsed / reps
    del payload, scales
    return {"us": round(s * 1e6, 1), "GBps": round(cw.algorithmic_bytes() / s / 1e9, 4), "reps": reps,
            "kept_tokens": cw.kept, "sample": "config 5 compaction in full (64 prefixes, out of place, payload + "
                                              "scales, L = 1), index_select + index_copy_"}


def _cpu_baseline(w, budget_s: float, torch, dev, workloads) -> dict:
    """CPU baselines on the GPU box's host cores: the headline decode sample
    (``value``) and configs 1, 2 (store) and 5 (compaction) as the reference's
    CPU paths run them, restated in ``oracle/``."""

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    dec = _cpu_decode_sample(w, 0.4 * budget_s, torch)
    configs = {
        "config1_decode_b1": _cpu_config1(dev, 0.15 * budget_s, torch, workloads),
        "config2_store": _cpu_store(dev, 0.25 * budget_s, torch, workloads),
        "config5_compaction": _cpu_compaction(0.2 * budget_s, torch, workloads),
    }
    return {
        "value": dec["GBps"],
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"first {dec['sequences']} of {w.batch} decode_mixed sequences, reference CPU path "
                  f"(page gather + bf16 dequant + GQA expand + SDPA), {dec['seconds']} s",
        "us_per_layer_equiv": dec["us_per_layer_equiv"],
        "configs": configs,
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=100)
    parser.add_argument("--layers", type=int, default=4, help="independent KV pools the steps rotate over")
    parser.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU baseline work")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-extras", action="store_true", help="skip store/compaction/single-sequence extras")
    parser.add_argument("--copy-probe", action="store_true",
                        help="only run a plain 1 GiB device copy (reference for rocprof FETCH/WRITE_SIZE scaling)")
    parser.add_argument("--store-probe", action="store_true",
                        help="only run the config-2 store, 8 calls over 8 distinct input chunks (target for rocprof "
                             "FETCH/WRITE_SIZE of the store kernel)")
    parser.add_argument("--compaction-probe", action="store_true",
                        help="only run the config-5 compaction (payload and scale calls) 3 times (target for rocprof "
                             "FETCH/WRITE_SIZE of the compaction kernels)")
    parser.add_argument("--prefill-probe", action="store_true",
                        help="only run the paged-prefill extra warm, 3 + 10 calls (target for rocprof statistics "
                             "and SQ counters of the prefill kernel)")
    args = parser.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the KV hot path needs no collective and this build "
              "runs no multi-GPU configuration (use --gpus 1).", file=sys.stderr)
        return 2

    import torch  # noqa: PLC0415

    from prism_infer import _native, workloads  # noqa: PLC0415
    from prism_infer.ops.paged_decode import (  # noqa: PLC0415
        _launch_paged_decode_attention,
        decode_workspace_bytes,
    )

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    _native.device_lib(torch.device("cuda", 0))
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.copy_probe:
        src = torch.ones(1 << 30, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_read": src.numel(), "copy_probe_bytes_written": dst.numel(), "calls": 5}))
        return 0

    if args.store_probe:
        from prism_infer.ops.kv_cache_store import store_kvcache  # noqa: PLC0415

        sw = workloads.store_prefill(dev)
        kc = torch.empty(sw.num_pages, 256, 8, 128, dtype=torch.float8_e4m3fn, device=dev)
        vc = torch.empty_like(kc)
        ks = torch.empty(sw.num_pages, 256, 8, dtype=torch.float32, device=dev)
        vs = torch.empty_like(ks)
        keys = [sw.key.roll(i, 0) for i in range(8)]
        values = [sw.value.roll(i, 0) for i in range(8)]
        torch.cuda.synchronize()
        for i in range(8):
            store_kvcache(keys[i], values[i], kc, vc, sw.slot_mapping, ks, vs)
        torch.cuda.synchronize()
        print(json.dumps({"store_probe_calls": 8, "algorithmic_bytes_per_call": sw.algorithmic_bytes()}))
        return 0

    if args.compaction_probe:
        from prism_infer.ops.kv_compaction import compact_kv_slots  # noqa: PLC0415

        cw = workloads.compaction_plans()
        slots = cw.num_pages * 256
        payload = torch.zeros(2, 1, slots, 8, 128, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
        scales = torch.zeros(2, 1, slots, 8, dtype=torch.float32, device=dev)
        src = torch.tensor([x for p in cw.plans for x in p.source_slots], dtype=torch.long, device=dev)
        dst = torch.tensor([x for p in cw.plans for x in p.destination_slots], dtype=torch.long, device=dev)
        torch.cuda.synchronize()
        for _ in range(3):
            compact_kv_slots(payload, src, dst)
            compact_kv_slots(scales, src, dst)
        torch.cuda.synchronize()
        print(json.dumps({"compaction_probe_calls": 3, "algorithmic_bytes_per_call": cw.algorithmic_bytes(),
                          "kept_tokens": cw.kept}))
        return 0

    if args.prefill_probe:
        from types import SimpleNamespace  # noqa: PLC0415

        from prism_infer.ops.paged_prefill import _launch_paged_prefill  # noqa: PLC0415

        pw = workloads.prefill_chunked(dev)
        pctx = SimpleNamespace(block_tables=pw.block_tables, context_lens=pw.context_lens,
                               cu_seqlens_q=pw.cu_seqlens_q)
        call = lambda i: _launch_paged_prefill(  # noqa: E731
            pw.q, pw.k_cache, pw.v_cache, pctx, num_heads=pw.num_heads, num_kv_heads=pw.num_kv_heads,
            scale=pw.scale, k_scale_cache=pw.k_scale, v_scale_cache=pw.v_scale)
        for i in range(3):
            call(i)
        s = _time_loop(call, 10, torch)
        print(json.dumps({"prefill_probe_us_warm": round(s * 1e6, 2), "TFLOPs": round(pw.flops() / s / 1e12, 1),
                          "mfma_frac": round(pw.flops() / s / MFMA_BF16_PEAK, 4), "calls": 13}))
        return 0

    # ---- headline workload: decode_mixed, one pool per rotated layer
    _log(f"building decode_mixed x {args.layers} layers")
    layers = []
    base = workloads.decode_mixed(dev)
    layers.append(base)
    for layer in range(1, args.layers):
        k, v, ks, vs = (torch.empty_like(t) for t in (base.k_cache, base.v_cache, base.k_scale, base.v_scale))
        workloads.fill_pages(k, v, ks, vs, base.used_pages, 1000 + layer)
        layers.append(type(base)(**{**base.__dict__, "k_cache": k, "v_cache": v, "k_scale": ks, "v_scale": vs}))
    torch.cuda.synchronize()
    alg_bytes = base.algorithmic_bytes()
    ws = torch.empty(max(decode_workspace_bytes(base.q, base.k_cache, base.block_tables), 1),
                     dtype=torch.uint8, device=dev)
    outs = [torch.empty_like(base.q) for _ in layers]

    def step(i: int, stage: int = 0):
        w = layers[i % len(layers)]
        _launch_paged_decode_attention(
            w.q, w.k_cache, w.v_cache, w.block_tables, w.context_lens, w.scale, w.max_context_len,
            k_scale_cache=w.k_scale, v_scale_cache=w.v_scale, scaled_kv=True, stage=stage,
            output=outs[i % len(layers)], workspace=ws)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    _log(f"timing {args.steps} steps")
    sec_per_step = _time_loop(step, args.steps, torch)
    # dominant kernel alone (stage 1: the streaming kernel, which checks the
    # plan in the workspace and merges its own partials -- the whole step),
    # same stream, same rotation
    for i in range(args.warmup):
        step(i, 1)
    kernel_s = _time_loop(lambda i: step(i, 1), args.steps, torch)

    value = alg_bytes / sec_per_step / 1e9
    achieved = alg_bytes / kernel_s / 1e9
    traffic = None
    if TRAFFIC_FILE.exists():
        try:
            traffic = json.loads(TRAFFIC_FILE.read_text()).get("hbm_bytes_per_launch")
        except (ValueError, OSError):
            traffic = None
    geo_args = (base.batch, 32, 8, 128, 256, base.block_tables.shape[1], 3)
    split = _native.lib().prism_paged_decode_split_tokens(*geo_args)
    family = _native.lib().prism_paged_decode_kernel_family(*geo_args)
    kernel_name = {2: "paged_decode_stream_kernel", 1: "paged_decode_split_kernel"}.get(family, "paged_decode_generic_kernel")
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(sec_per_step * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "decode_mixed: batch 64, context U[1024,16384] (seeded), 32 sequences share a "
                        "4096-token prefix (16 pages), 32q/8kv heads, head_dim 128, 256-token scaled-FP8 "
                        "pages in an 8192-page pool; one step = one layer's decode",
            "batch": base.batch,
            "context_lens_sum": int(base.context_lens.sum().item()),
            "unique_kv_tokens": base.unique_kv_tokens(),
            "algorithmic_bytes_per_step": alg_bytes,
            "layers_rotated": len(layers),
            "split_tokens": int(split),
        },
        "us_per_layer": round(sec_per_step * 1e6, 2),
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBPS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "kernel": kernel_name,
            "kernel_us": round(kernel_s * 1e6, 2),
            "rest_of_step_us": round((sec_per_step - kernel_s) * 1e6, 2),
        },
    }

    if not args.no_extras:
        result["decode_step_graph"] = _graph_steps(step, 36, outs, alg_bytes, torch)
        result["decode_tp_shards"] = {f"tp{tp}": _tp_shard(layers, torch, tp) for tp in (2, 4, 8)}
        result["extras"] = _extras(torch, dev, workloads)
    del layers, outs, ws
    torch.cuda.empty_cache()

    if not args.no_cpu_baseline:
        _log("cpu baseline")
        result["cpu_baseline"] = _cpu_baseline(base, args.cpu_budget, torch, dev, workloads)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


def _check_long_sample(lw, out, torch) -> dict:
    """Compare two sequences of the chained config-5 decode (one starting with
    a compacted prefix, one private) with the CPU oracle, pages copied only."""

    import oracle  # noqa: PLC0415  (checker only)

    rows = torch.tensor([0, lw.batch - 1])
    tables = lw.block_tables.cpu().to(torch.int64)[rows]
    pages = torch.unique(tables[tables >= 0])
    remap = torch.full((lw.k_cache.shape[0],), -1, dtype=torch.int64)
    remap[pages] = torch.arange(pages.numel())
    local = torch.where(tables >= 0, remap[tables.clamp(min=0)], tables).to(torch.int32)
    idx = pages.to(lw.k_cache.device)
    k = lw.k_cache.view(torch.uint8).index_select(0, idx).cpu().view(torch.float8_e4m3fn)
    v = lw.v_cache.view(torch.uint8).index_select(0, idx).cpu().view(torch.float8_e4m3fn)
    ks, vs = lw.k_scale.index_select(0, idx).cpu(), lw.v_scale.index_select(0, idx).cpu()
    want = oracle.decode_kernel_semantics(lw.q.cpu()[rows], k, v, local, lw.context_lens.cpu()[rows], lw.scale,
                                          k_scale_cache=ks, v_scale_cache=vs, compute_dtype=torch.float32)
    got = out.cpu()[rows].float()
    err = (got - want.float()).abs()
    bound = 2e-2 + 1e-2 * want.float().abs()
    return {"sequences": rows.tolist(), "max_abs_err": round(float(err.max()), 6),
            "within_tolerance": bool(torch.all(err <= bound))}


def _tp_shard(layers, torch, tp: int, steps: int = 50) -> dict:
    """One tensor-parallel rank's share of the headline step at TP = tp: the
    same sequences and pages with the first 8 / tp of the 8 kv heads (a
    contiguous cache of that many heads, Hq = 32 / tp), one streaming launch
    per step.  Timed as the headline is: the steps rotate over the rotated
    layer pools' shards (each step reads a shard the previous steps did not),
    HIP events around `steps` eager steps; `warm_us_per_layer` repeats one
    pool's shard (at TP 8 a shard is 125 MB, which the 256 MB MALL holds)."""

    from prism_infer import _native  # noqa: PLC0415
    from prism_infer.ops.paged_decode import (  # noqa: PLC0415
        _launch_paged_decode_attention,
        decode_workspace_bytes,
    )

    base = layers[0]
    hkv, hq = 8 // tp, 32 // tp
    q = base.q[:, :hq].contiguous()
    shards = [tuple(t[:, :, :hkv].contiguous() for t in (w.k_cache, w.v_cache, w.k_scale, w.v_scale)) for w in layers]
    ws = torch.empty(decode_workspace_bytes(q, shards[0][0], base.block_tables), dtype=torch.uint8, device=q.device)
    out = torch.empty_like(q)

    def call(i, stage=0, rotate=True):
        k, v, ks, vs = shards[i % len(shards)] if rotate else shards[0]
        _launch_paged_decode_attention(q, k, v, base.block_tables, base.context_lens, base.scale,
                                       base.max_context_len, k_scale_cache=ks, v_scale_cache=vs, scaled_kv=True,
                                       stage=stage, output=out, workspace=ws)

    for i in range(steps):
        call(i)
    s = _time_loop(call, steps, torch)
    kernel = _time_loop(lambda i: call(i, 1), steps, torch)
    warm = _time_loop(lambda i: call(i, 0, False), steps, torch)
    family = _native.lib().prism_paged_decode_kernel_family(base.batch, hq, hkv, 128, 256, base.block_tables.shape[1],
                                                            3)
    k, v, ks, vs = shards[0]
    shard = type(base)(**{**base.__dict__, "q": q, "k_cache": k, "v_cache": v, "k_scale": ks, "v_scale": vs})
    shard_bytes = shard.algorithmic_bytes()
    del shards, ws, shard
    return {"us_per_layer": round(s * 1e6, 2), "GBps": round(shard_bytes / s / 1e9, 1),
            "pct_of_hbm_peak": round(100.0 * shard_bytes / s / 1e9 / HBM_PEAK_GBPS, 2),
            "kernel_us": round(kernel * 1e6, 2), "warm_us_per_layer": round(warm * 1e6, 2),
            "kernel_family": int(family), "kv_heads": hkv, "q_heads": hq, "layers_rotated": len(layers),
            "timing": "eager, HIP events, steps rotating over the layer pools' shards as the headline does"}


def _graph_steps(step, n_layers: int, outs, alg_bytes: int, torch, reps: int = 8, warm: int = 6) -> dict:
    """The headline step for ``n_layers`` layers (one decode step of a
    36-layer model; the layers cycle over the rotated pools) captured once in
    a HIP graph and replayed, as a serving engine runs decode: no host launch
    gaps between the kernels.  ``warm`` replays run untimed first (the first
    replays after a capture ran up to 30% slower on this stack).  The last
    replay's outputs are checked against an eager run of the same layers."""

    for i in range(n_layers):
        step(i)
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs[:n_layers]]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(n_layers):
            step(i)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(n_layers):
            step(i)
    for _ in range(warm):
        graph.replay()
    torch.cuda.synchronize()
    s = _time_loop(lambda i: graph.replay(), reps, torch) / n_layers
    same = all(torch.equal(o, e) for o, e in zip(outs[:n_layers], eager))
    return {"us_per_layer": round(s * 1e6, 2), "GBps": round(alg_bytes / s / 1e9, 1),
            "pct_of_hbm_peak": round(100.0 * alg_bytes / s / 1e9 / HBM_PEAK_GBPS, 2),
            "replays": reps, "layers_per_graph": n_layers, "matches_eager": same,
            "timing": "warm, HIP events around graph replays"}


def _extras(torch, dev, workloads) -> dict:
    """GPU time of the other configurations: store (config 2), compaction
    (config 5), B = 1 decode over 36 layers (config 3), the config-5 chain,
    paged prefill, a batch of copy-on-write block copies and config 4's
    decode over unit-scale FP8 and bf16 caches.  Each runs after a 1 GiB
    write that evicts the MALL and L2 ("cold"), queued behind a GPU spin so
    that only GPU time is measured (``_time_queued``)."""

    from prism_infer.engine.kv_block_ops import copy_kv_blocks  # noqa: PLC0415
    from prism_infer.ops.kv_cache_store import store_kvcache  # noqa: PLC0415
    from prism_infer.ops.kv_compaction import compact_kv_slots  # noqa: PLC0415
    from prism_infer.ops.paged_decode import paged_decode_attention  # noqa: PLC0415

    scratch = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    flush = lambda: scratch.fill_(1)
    out = {}
    # The queued timing of one call has a fixed floor (the start event, then
    # the launch): measure it with a one-element kernel, to read short calls.
    tiny = torch.zeros(1, device=dev)
    out["queued_call_floor_us"] = round(_time_queued(lambda i: tiny.add_(1), 1, torch, flush=flush) * 1e6, 2)
    out["copy_ceiling"] = _copy_ceiling(torch, dev, flush)
    # store: 8192 tokens into a 512-page pool; one call cold, and 8 calls back
    # to back over 8 distinct input chunks (268 MB, more than the MALL), as a
    # prefill's layers issue them
    sw = workloads.store_prefill(dev)
    kc = torch.empty(sw.num_pages, 256, 8, 128, dtype=torch.float8_e4m3fn, device=dev)
    vc = torch.empty_like(kc)
    ks = torch.empty(sw.num_pages, 256, 8, dtype=torch.float32, device=dev)
    vs = torch.empty_like(ks)
    s1 = _time_queued(lambda i: store_kvcache(sw.key, sw.value, kc, vc, sw.slot_mapping, ks, vs), 1, torch,
                      flush=flush)
    keys = [sw.key.roll(i, 0) for i in range(8)]
    values = [sw.value.roll(i, 0) for i in range(8)]
    s8 = _time_queued(lambda i: store_kvcache(keys[i], values[i], kc, vc, sw.slot_mapping, ks, vs), 8, torch,
                      flush=flush)
    # warm: the inputs resident in the MALL, as right after the QKV projection
    # wrote them (8 calls over one 33.5 MB input chunk, no flush)
    store_kvcache(keys[0], values[0], kc, vc, sw.slot_mapping, ks, vs)
    sw8 = _time_queued(lambda i: store_kvcache(keys[0], values[0], kc, vc, sw.slot_mapping, ks, vs), 8, torch)
    out["store_prefill"] = {"us": round(s8 * 1e6, 2), "GBps": round(sw.algorithmic_bytes() / s8 / 1e9, 1),
                            "pct_of_hbm_peak": round(100.0 * sw.algorithmic_bytes() / s8 / 1e9 / HBM_PEAK_GBPS, 2),
                            "frac_of_copy_ceiling": round(sw.algorithmic_bytes() / s8 / 1e9 /
                                                          out["copy_ceiling"]["best_store_size_GBps"], 4),
                            "us_single_call": round(s1 * 1e6, 2), "us_warm_inputs": round(sw8 * 1e6, 2),
                            "bytes": sw.algorithmic_bytes(),
                            "timing": "8 calls back to back over 8 distinct cold input chunks, queued behind a "
                                      "spin (us_single_call: one cold call, including the queued-call floor; "
                                      "us_warm_inputs: 8 calls over one input chunk resident in the MALL)"}
    del kc, vc, ks, vs, keys, values
    # compaction: 64 x 8192-token prefixes, ~30% dropped, out of place, payload + scales (L=1)
    cw = workloads.compaction_plans()
    slots = cw.num_pages * 256
    payload = torch.zeros(2, 1, slots, 8, 128, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    scales = torch.zeros(2, 1, slots, 8, dtype=torch.float32, device=dev)
    src = torch.tensor([x for p in cw.plans for x in p.source_slots], dtype=torch.long, device=dev)
    dst = torch.tensor([x for p in cw.plans for x in p.destination_slots], dtype=torch.long, device=dev)

    def compact(i):
        compact_kv_slots(payload, src, dst)
        compact_kv_slots(scales, src, dst)

    s = _time_queued(compact, 1, torch, flush=flush)
    copy_gbps = out["copy_ceiling"]["best_GBps"]
    out["compaction_out_of_place"] = {"us": round(s * 1e6, 2), "GBps": round(cw.algorithmic_bytes() / s / 1e9, 1),
                                      "bytes": cw.algorithmic_bytes(), "kept_tokens": cw.kept,
                                      "pct_of_hbm_peak": round(100.0 * cw.algorithmic_bytes() / s / 1e9 /
                                                               HBM_PEAK_GBPS, 2),
                                      "copy_ceiling_GBps": round(copy_gbps, 1),
                                      "frac_of_copy_ceiling": round(cw.algorithmic_bytes() / s / 1e9 / copy_gbps, 4),
                                      "timing": "queued behind a spin, cold (payload and scale calls); copy "
                                                "ceiling: the copy_ceiling extra"}
    del payload, scales, src, dst
    # single-sequence decode (latency bound): Qwen3-VL-shaped, B=1, 1800 tokens, 36 layers with their own pools
    layers = [workloads.decode_qwen_vl(dev, seed=20260803 + li) for li in range(36)]
    s = _time_queued(lambda i: paged_decode_attention(
        layers[i].q, layers[i].k_cache, layers[i].v_cache, layers[i].block_tables, layers[i].context_lens,
        layers[i].scale, k_scale_cache=layers[i].k_scale, v_scale_cache=layers[i].v_scale,
        max_context_len=layers[i].max_context_len), 36, torch, flush=flush)
    out["decode_qwen_vl_b1"] = {"us_per_layer": round(s * 1e6, 2),
                                "GBps": round(layers[0].algorithmic_bytes() / s / 1e9, 1),
                                "timing": "36 layers back to back, queued behind a spin, cold"}
    del layers
    # config 5 as a chain: compaction of 64 prefixes into dense pages, then
    # decode of B = 256 at 32k tokens each (sequences 0..63 start with their
    # compacted prefix pages), pages scattered in a ~120 GB pool
    lw = workloads.decode_long_compacted(dev, pool_pages=LONG_POOL_PAGES)
    call = lambda i: paged_decode_attention(
        lw.q, lw.k_cache, lw.v_cache, lw.block_tables, lw.context_lens, lw.scale, k_scale_cache=lw.k_scale,
        v_scale_cache=lw.v_scale, max_context_len=lw.max_context_len)
    s = _time_queued(call, 3, torch, flush=flush)
    check = _check_long_sample(lw, call(0), torch)
    pool_bytes = sum(t.numel() * t.element_size() for t in (lw.k_cache, lw.v_cache, lw.k_scale, lw.v_scale))
    out["decode_long_b256"] = {"us": round(s * 1e6, 1), "GBps": round(lw.algorithmic_bytes() / s / 1e9, 1),
                               "pct_of_hbm_peak": round(100.0 * lw.algorithmic_bytes() / s / 1e9 / HBM_PEAK_GBPS, 2),
                               "bytes": lw.algorithmic_bytes(), "pool_GB": round(pool_bytes / 1e9, 1),
                               "compacted_prefixes": lw.meta["compacted"],
                               "compacted_kept_tokens": lw.meta["compaction"].kept, "check": check,
                               "timing": "3 calls back to back, queued behind a spin, cold"}
    del lw
    # paged prefill: 4 sequences x (8192 cached + 2048 new tokens), causal
    from types import SimpleNamespace  # noqa: PLC0415

    from prism_infer.ops.paged_prefill import _launch_paged_prefill  # noqa: PLC0415

    pw = workloads.prefill_chunked(dev)
    pctx = SimpleNamespace(block_tables=pw.block_tables, context_lens=pw.context_lens, cu_seqlens_q=pw.cu_seqlens_q)
    s = _time_queued(lambda i: _launch_paged_prefill(
        pw.q, pw.k_cache, pw.v_cache, pctx, num_heads=pw.num_heads, num_kv_heads=pw.num_kv_heads, scale=pw.scale,
        k_scale_cache=pw.k_scale, v_scale_cache=pw.v_scale), 1, torch, flush=flush)
    out["prefill_chunked"] = {"us": round(s * 1e6, 2), "TFLOPs": round(pw.flops() / s / 1e12, 1),
                              "mfma_frac": round(pw.flops() / s / MFMA_BF16_PEAK, 4), "flops": pw.flops(),
                              "GBps": round(pw.algorithmic_bytes() / s / 1e9, 1),
                              "timing": "queued behind a spin, cold (status fill + kernel; the host check is not timed)"}
    del pw
    # copy-on-write: 128 block pairs of a [2, 4, 1024, 256, 8, 128] cache, payload and scales
    cache = torch.zeros(2, 4, 1024, 256, 8, 128, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    scache = torch.zeros(2, 4, 1024, 256, 8, dtype=torch.float32, device=dev)
    pairs = [(i, 512 + i) for i in range(128)]
    nbytes = 2 * len(pairs) * 2 * 4 * 256 * 8 * (128 + 4)
    copy_kv_blocks(cache, pairs, scache)  # the API once; the timed calls reuse its device index tensors
    bsrc = torch.tensor([p[0] for p in pairs], dtype=torch.long, device=dev)
    bdst = torch.tensor([p[1] for p in pairs], dtype=torch.long, device=dev)

    def cow(i):
        compact_kv_slots(cache.view(2, 4, 1024, -1), bsrc, bdst)
        compact_kv_slots(scache.view(2, 4, 1024, -1), bsrc, bdst)

    s = _time_queued(cow, 1, torch, flush=flush)
    out["copy_on_write_blocks"] = {"us": round(s * 1e6, 2), "GBps": round(nbytes / s / 1e9, 1), "bytes": nbytes,
                                   "pairs": len(pairs), "layers": 4, "timing": "queued behind a spin, cold"}
    del scache
    # the dense variants of config 4's decode (same sequences, tables and
    # pages): a unit-scale FP8 cache (no scale caches) and a bf16 cache (the
    # dequantised pages), both on the split-K kernel, which reads each
    # sequence's pages (shared ones included) once per sequence
    w = workloads.decode_mixed(dev)
    attended = int(w.context_lens.sum().item())
    unique = w.unique_kv_tokens()
    fixed = w.algorithmic_bytes() - unique * 2112  # q, output, tables, lengths
    variants = {}
    for name, k, v, row in (("unit_scale_fp8", w.k_cache, w.v_cache, 2 * 8 * 128),
                            ("bf16", (w.k_cache.float() * w.k_scale.unsqueeze(-1)).to(torch.bfloat16),
                             (w.v_cache.float() * w.v_scale.unsqueeze(-1)).to(torch.bfloat16), 2 * 8 * 128 * 2)):
        call = lambda i, k=k, v=v: paged_decode_attention(  # noqa: E731
            w.q, k, v, w.block_tables, w.context_lens, w.scale, max_context_len=w.max_context_len)
        s = _time_queued(call, 3, torch, flush=flush)
        alg = unique * row + fixed
        variants[name] = {"us": round(s * 1e6, 1), "GBps": round(alg / s / 1e9, 1),
                          "pct_of_hbm_peak": round(100.0 * alg / s / 1e9 / HBM_PEAK_GBPS, 2), "bytes": alg,
                          "GBps_attended": round(attended * row / s / 1e9, 1), "bytes_attended": attended * row}
        del k, v
    out["decode_mixed_dense_variants"] = {
        **variants, "timing": "3 calls back to back, queued behind a spin, cold",
        "bytes_note": "bytes: each unique (page, row) once (the shared prefix once) + q, output, tables, lengths; "
                      "bytes_attended counts the shared prefix once per sequence"}
    del w
    out["decode_small_batch_matrix"] = _small_batch_matrix(torch, dev, flush)
    return out


def _copy_ceiling(torch, dev, flush) -> dict:
    """Read + write ceiling of a plain device copy, cold: torch's Tensor.copy_
    of 1 GiB, and the library's streaming copy (prism_device_copy: persistent
    grid, non-temporal 16-byte loads and stores, eight in flight per lane) at
    1, 2, 4 and 8 workgroups per CU, over 1 GiB (one call) and over the store's
    size (25.4 MB read + 25.4 MB written, 8 calls back to back over 8 distinct
    buffers, as the store extra is timed)."""

    from prism_infer import _native  # noqa: PLC0415

    lib = _native.device_lib(dev)
    stream = _native.stream_handle(dev)
    res = {}
    for nbytes, calls, tag in ((1 << 30, 1, "1GiB"), (25_444_352, 8, "store_size")):
        srcs = [torch.ones(nbytes, dtype=torch.uint8, device=dev) for _ in range(calls)]
        dsts = [torch.empty_like(x) for x in srcs]
        sec = _time_queued(lambda i: dsts[i].copy_(srcs[i]), calls, torch, flush=flush)
        res[f"torch_copy_{tag}_GBps"] = round(2 * nbytes / sec / 1e9, 1)
        for wpc in (1, 2, 4, 8):
            call = lambda i, w=wpc: _native.check(  # noqa: E731
                lib.prism_device_copy(dsts[i].data_ptr(), srcs[i].data_ptr(), nbytes, w, stream),
                "prism_device_copy")
            sec = _time_queued(call, calls, torch, flush=flush)
            res[f"stream_copy_{tag}_wpc{wpc}_GBps"] = round(2 * nbytes / sec / 1e9, 1)
            res[f"stream_copy_{tag}_wpc{wpc}_us"] = round(sec * 1e6, 2)
        assert all(torch.equal(d, x) for d, x in zip(dsts, srcs))
        del srcs, dsts
    res["best_GBps"] = max(v for k, v in res.items() if "1GiB" in k and k.endswith("GBps"))
    res["best_store_size_GBps"] = max(v for k, v in res.items() if "store_size" in k and k.endswith("GBps"))
    res["timing"] = "queued behind a spin, cold; GBps = 2 x bytes (read + write) / time per call"
    return res


def _small_batch_matrix(torch, dev, flush) -> dict:
    """The reference's kernel benchmark matrix (benchmarks/bench_paged_decode.py:40-51):
    B in {1, 2, 4, 8} x context in {256, 1024, 4096} tokens, 32 q / 8 kv heads,
    head_dim 128, 256-token pages, bf16 queries; caches bf16, unit-scale FP8
    (the reference harness's "fp8": a cast, no scales) and scaled FP8.  Each
    shape runs as 8 layers with their own pools, back to back, cold (the
    reference times one warm call with host timers)."""

    from prism_infer.ops.kv_cache_store import store_kvcache  # noqa: PLC0415
    from prism_infer.ops.paged_decode import paged_decode_attention  # noqa: PLC0415

    layers, page, hq, hkv, d = 8, 256, 32, 8, 128
    g = torch.Generator(device=dev)
    g.manual_seed(20260717)
    rows = {}
    for ctx in (256, 1024, 4096):
        for batch in (1, 2, 4, 8):
            pages = -(-ctx // page)
            tables = torch.arange(batch * pages, dtype=torch.int32, device=dev).view(batch, pages)
            lens = torch.full((batch,), ctx, dtype=torch.int32, device=dev)
            q = torch.randn(batch, hq, d, generator=g, device=dev, dtype=torch.bfloat16)
            slots = torch.arange(batch * pages * page, dtype=torch.int32, device=dev).view(batch, -1)[:, :ctx]
            slots = slots.reshape(-1).contiguous()
            dense, unit, scaled = [], [], []
            for _ in range(layers):
                kd = torch.zeros(batch * pages, page, hkv, d, dtype=torch.bfloat16, device=dev)
                vd = torch.zeros_like(kd)
                key = torch.randn(batch * ctx, hkv, d, generator=g, device=dev, dtype=torch.bfloat16)
                val = torch.randn(batch * ctx, hkv, d, generator=g, device=dev, dtype=torch.bfloat16)
                store_kvcache(key, val, kd, vd, slots)
                dense.append((kd, vd, None, None))
                unit.append((kd.to(torch.float8_e4m3fn), vd.to(torch.float8_e4m3fn), None, None))
                k8 = torch.zeros(batch * pages, page, hkv, d, dtype=torch.float8_e4m3fn, device=dev)
                v8 = torch.zeros_like(k8)
                ks = torch.zeros(batch * pages, page, hkv, dtype=torch.float32, device=dev)
                vs = torch.zeros_like(ks)
                store_kvcache(key, val, k8, v8, slots, ks, vs)
                scaled.append((k8, v8, ks, vs))
            fixed = 2 * batch * hq * d * 2 + batch * pages * 4 + batch * 4
            for name, caches, per_tok in (("bf16", dense, 2 * hkv * d * 2), ("fp8", unit, 2 * hkv * d),
                                          ("scaled_fp8", scaled, 2 * hkv * d + 2 * hkv * 4)):
                call = lambda i, c=caches: paged_decode_attention(  # noqa: E731
                    q, c[i][0], c[i][1], tables, lens, d ** -0.5, k_scale_cache=c[i][2], v_scale_cache=c[i][3])
                sec = _time_queued(call, layers, torch, flush=flush)
                alg = batch * ctx * per_tok + fixed
                rows[f"{name}_b{batch}_ctx{ctx}"] = {"us": round(sec * 1e6, 2), "GBps": round(alg / sec / 1e9, 1)}
            del dense, unit, scaled
    return {**rows, "timing": "8 layers back to back per shape, queued behind a spin, cold; GBps: unique K/V "
                              "(+ scales) + q + output + tables + lengths per call"}


if __name__ == "__main__":
    sys.exit(main())
