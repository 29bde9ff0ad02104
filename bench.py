#!/usr/bin/env python3
"""Headline benchmark: Qwen2.5-7B-shape paged decode on one MI355X.

One step = one layer's hot path over the batch: the slot-mapped append of one
new K/V token per sequence (fused into the decode kernel), split-K paged decode
attention and the merge of its partials, through the backend API, on
seeded synthetic bf16 pools (64 sequences, contexts U[512, 4096], random
non-overlapping block tables from a 32768-block pool, 28 Q / 4 KV heads,
head_size 128, block_size 16).

* ``value``      GB/s = algorithmic bytes per step / measured step time
  (KV rows read once + Q + O + block tables + append read/write), with inputs
  resident in HBM.  Several independent pool sets rotate step by step so the
  256 MB Infinity Cache cannot serve a step from the previous one.
* ``roofline``   the decode kernel alone: algorithmic bytes per launch / its
  mean launch time from HIP events on the launch stream (batches of
  back-to-back launches), against 8 TB/s; ``traffic`` is the HBM bytes per
  launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE runs.
* ``cpu_baseline`` the CPU oracle (numpy restatement of light-vllm's Torch
  paged attention + index_copy append) on the same step, on this host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--sets R]
"""

from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
importlib.import_module("light-vllm_amd")
import light_vllm_amd as lv  # noqa: E402

METRIC = "paged-decode HBM GB/s (% of peak) + tokens/s, Qwen2.5-7B shape bs64"
HBM_PEAK_GBS = 8000.0
NUM_LAYERS = 28  # Qwen2.5-7B: tokens/s = batch / (28 * t_layer), attention-only


class C2:
    hq, hkv, d, bs, num_blocks, batch = 28, 4, 128, 16, 32768, 64
    ctx_lo, ctx_hi = 512, 4096
    dtype = torch.bfloat16
    seed = 20261201


def build_workload(num_sets: int, device: torch.device):
    cfg = C2
    rng = np.random.default_rng(cfg.seed)
    ctx = rng.integers(cfg.ctx_lo, cfg.ctx_hi + 1, size=cfg.batch)
    need = (ctx + 1 + cfg.bs - 1) // cfg.bs
    perm = rng.permutation(cfg.num_blocks)
    tables, off = [], 0
    for n in need:
        tables.append(tuple(int(b) for b in perm[off : off + n]))
        off += int(n)
    metadata = lv.PagedAttentionMetadata(
        block_tables=tuple(tables),
        num_computed_tokens=tuple(int(c) for c in ctx),
        query_layouts=tuple(lv.linear_query_layout(1) for _ in range(cfg.batch)),
    )
    spec = lv.ModelKVCacheSpec((lv.AttentionLayerSpec("layer0", cfg.hq, cfg.hkv, cfg.d),))
    config = lv.PagedKVCacheConfig(num_blocks=cfg.num_blocks, block_size=cfg.bs, dtype=cfg.dtype, device=device)
    gen = torch.Generator(device=device).manual_seed(cfg.seed)
    caches = []
    for _ in range(num_sets):
        cache = lv.PagedKVCache(spec, config)
        layer = cache.layer("layer0")
        for pool in (layer.keys, layer.values):
            pool.copy_(torch.randn(pool.shape, generator=gen, device=device, dtype=torch.float32).to(cfg.dtype))
        caches.append(cache)
    q = torch.randn((cfg.batch, cfg.hq, cfg.d), generator=gen, device=device).to(cfg.dtype)
    k = torch.randn((cfg.batch, cfg.hkv, cfg.d), generator=gen, device=device).to(cfg.dtype)
    v = torch.randn((cfg.batch, cfg.hkv, cfg.d), generator=gen, device=device).to(cfg.dtype)
    return metadata, caches, q, k, v, ctx


def algorithmic_bytes(ctx: np.ndarray) -> dict:
    cfg = C2
    s = 2  # bf16
    L = ctx + 1
    kv = int(L.sum()) * 2 * cfg.hkv * cfg.d * s
    q = o = cfg.batch * cfg.hq * cfg.d * s
    tables = int(((L + cfg.bs - 1) // cfg.bs).sum()) * 4
    append = 4 * cfg.batch * cfg.hkv * cfg.d * s
    flops = 4 * cfg.hq * cfg.d * int(L.sum())
    return {"kv": kv, "q": q, "o": o, "tables": tables, "append": append,
            "step": kv + q + o + tables + append, "decode": kv + q + o + tables, "flops": flops}


def cpu_baseline(metadata, cache, q, k, v, ctx, budget_s: float) -> dict:
    """Time the CPU oracle (append + per-query online softmax) on the same step."""

    from oracle import paged_kv_oracle as O  # checker/baseline only

    layer = cache.layer("layer0")
    used = sorted({b for t in metadata.block_tables for b in t})
    remap = {b: i for i, b in enumerate(used)}
    idx = torch.tensor(used, dtype=torch.long, device=layer.keys.device)
    kpool = layer.keys.index_select(0, idx).float().cpu().numpy()
    vpool = layer.values.index_select(0, idx).float().cpu().numpy()
    tables = [tuple(remap[b] for b in t) for t in metadata.block_tables]
    slots = O.slot_mapping(tables, list(metadata.num_computed_tokens), [1] * len(tables), [1] * len(tables), C2.bs)
    qn, kn, vn = q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy()
    parents = [(-1,)] * len(tables)
    scale = 1.0 / math.sqrt(C2.d)
    times = []
    start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        O.append(kpool, vpool, kn, vn, slots)
        O.paged_attention(qn, kpool, vpool, tables, list(metadata.num_computed_tokens), parents, scale=scale)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - start >= budget_s or len(times) >= 50:
            break
    step_s = float(np.mean(times))
    return {
        "value": round(algorithmic_bytes(ctx)["step"] / step_s / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"full C2 step (64 seqs, 1 layer) x{len(times)}, mean {step_s * 1e3:.1f} ms/step, "
                  f"numpy oracle, single thread, host {os.cpu_count()} cpus",
    }


def copy_calibration(args, device: torch.device) -> int:
    """A plain device-to-device copy of 1 GiB: counter calibration and practical ceiling."""

    nbytes = 1 << 30
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device=device) for _ in range(4)]
    for b in bufs:
        b.fill_(1)
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for i in range(args.warmup):
        bufs[(2 * i + 1) % 4].copy_(bufs[(2 * i) % 4])
    stream = torch.cuda.current_stream(device)
    for i, (a, b) in enumerate(events):
        a.record(stream)
        bufs[(2 * i + 1) % 4].copy_(bufs[(2 * i) % 4])
        b.record(stream)
    torch.cuda.synchronize()
    ms = float(np.mean([a.elapsed_time(b) for a, b in events]))
    gbs = 2 * nbytes / (ms * 1e-3) / 1e9
    # Read-only ceiling: a float32 sum over 1 GiB (reduction writes ~nothing).
    sums = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    views = [b.view(torch.float32) for b in bufs]
    for i in range(args.warmup):
        views[i % 4].sum()
    for i, (a, b) in enumerate(sums):
        a.record(stream)
        views[i % 4].sum()
        b.record(stream)
    torch.cuda.synchronize()
    read_ms = float(np.mean([a.elapsed_time(b) for a, b in sums]))
    read_gbs = nbytes / (read_ms * 1e-3) / 1e9
    print(json.dumps({"mode": "copy", "bytes_read": nbytes, "bytes_written": nbytes, "ms_per_copy": round(ms, 4),
                      "read_plus_write_GBps": round(gbs, 1), "frac_of_8TBps": round(gbs / HBM_PEAK_GBS, 4),
                      "read_only_ms": round(read_ms, 4), "read_only_GBps": round(read_gbs, 1)}),
          flush=True)
    return 0


TRAFFIC_SUMMARY = Path(__file__).resolve().parent / "profiles" / "paged_decode_c2_traffic.json"


def measured_traffic() -> dict | None:
    """HBM bytes per decode launch from the committed rocprofv3 counter runs.

    FETCH_SIZE and WRITE_SIZE (KiB per dispatch) of the decode kernel, each
    scaled by what the same counter reads for a plain copy of known size
    (the summary file records both runs and the factors).
    """

    if not TRAFFIC_SUMMARY.exists():
        return None
    summary = json.loads(TRAFFIC_SUMMARY.read_text())
    return {"bytes_per_launch": summary["hbm_bytes_per_launch"], "source": TRAFFIC_SUMMARY.name}


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--sets", type=int, default=4, help="rotating pool sets (1 GiB each)")
    parser.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU-baseline work")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--mode", choices=("full", "decode", "copy"), default="full",
                        help="decode: only the decode kernel (counter runs); copy: a plain 1 GiB device "
                             "copy of known size (counter calibration and the practical HBM ceiling)")
    parser.add_argument("--partition", type=int, default=None,
                        help="cap on the tokens one decode wave handles (default: spread over all resident waves)")
    args = parser.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the paged-KV path would shard by sequence or KV head with no exchange).", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X GPU", file=sys.stderr)
        return 1
    device = torch.device("cuda:0")
    if args.mode == "copy":
        return copy_calibration(args, device)
    print(f"[bench] building C2 workload, {args.sets} pool sets", file=sys.stderr, flush=True)
    metadata, caches, q, k, v, ctx = build_workload(args.sets, device)
    nbytes = algorithmic_bytes(ctx)
    backend = lv.HipPagedAttentionBackend(partition_tokens=args.partition)
    out = torch.empty_like(q)

    def step(i: int) -> torch.Tensor:
        cache = caches[i % len(caches)]
        return backend.create(cache, metadata).forward("layer0", q, k, v, scale=1.0 / math.sqrt(C2.d))

    launches = []
    for cache in caches:
        ctx_obj = backend.create(cache, metadata)
        launches.append(ctx_obj.decode_launch("layer0", q, out, scale=1.0 / math.sqrt(C2.d)))

    if args.mode == "decode":
        for i in range(args.warmup + args.steps):
            launches[i % len(launches)].decode()
        torch.cuda.synchronize()
        print(f"[bench] decode-only launches done: {args.warmup + args.steps}", file=sys.stderr, flush=True)
        return 0

    # End-to-end steps.
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    print(f"[bench] warmup done ({args.warmup} steps)", file=sys.stderr, flush=True)
    t0 = time.perf_counter()
    for i in range(args.steps):
        result = step(i)
    submitted = time.perf_counter() - t0
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed / args.steps * 1e3
    assert torch.isfinite(result.float()).all()
    print(f"[bench] timed {args.steps} steps: {ms_per_step:.4f} ms/step "
          f"(host submit {submitted / args.steps * 1e3:.4f} ms/step)", file=sys.stderr, flush=True)

    # Decode kernel alone: HIP events on the launch stream (torch's current
    # stream) around batches of back-to-back launches, rotating pool sets.
    stream = torch.cuda.current_stream(device)
    batch = 10
    rounds = max(1, args.steps // batch)
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(rounds)]
    for i in range(args.warmup):
        launches[i % len(launches)].decode()
    for r, (a, b) in enumerate(events):
        a.record(stream)
        for i in range(batch):
            launches[(r * batch + i) % len(launches)].decode()
        b.record(stream)
    torch.cuda.synchronize()
    durations = np.array([a.elapsed_time(b) for a, b in events]) / batch  # ms per launch
    decode_ms = float(durations.mean())
    achieved = nbytes["decode"] / (decode_ms * 1e-3) / 1e9
    print(f"[bench] decode kernel: mean {decode_ms * 1e3:.2f} us over {rounds} x {batch} launches, "
          f"p10 {np.percentile(durations, 10) * 1e3:.2f}, p90 {np.percentile(durations, 90) * 1e3:.2f}",
          file=sys.stderr, flush=True)

    value = nbytes["step"] / (ms_per_step * 1e-3) / 1e9
    record = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) bf16 KV pools, random non-overlapping block tables",
        "config": {
            "workload": "C2 Qwen2.5-7B-shape paged decode, one layer: append 1 token/seq + split-K attention",
            "batch": C2.batch, "q_heads": C2.hq, "kv_heads": C2.hkv, "head_size": C2.d, "block_size": C2.bs,
            "pool_blocks": C2.num_blocks, "context": f"U[{C2.ctx_lo},{C2.ctx_hi}] seed {C2.seed}",
            "mean_context": float(ctx.mean()), "rotating_pool_sets": len(caches),
            "decode_waves": launches[0].work.waves_per_head * C2.hkv if launches[0] else None,
            "tiles_per_wave": launches[0].work.tiles_per_wave if launches[0] else None,
        },
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "tokens_per_s": round(C2.batch / (NUM_LAYERS * ms_per_step * 1e-3), 1),
        "tokens_per_s_note": "attention-only: batch / (28 layers x step time)",
        "algorithmic_bytes_per_step": nbytes["step"],
        "decode_kernel_us": round(decode_ms * 1e3, 3),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "paged_decode_kernel<bf16,128>",
            "algorithmic_bytes_per_launch": nbytes["decode"],
        },
    }
    traffic = measured_traffic()
    if traffic is not None:
        record["roofline"]["traffic"] = traffic["bytes_per_launch"]
        record["roofline"]["traffic_source"] = traffic["source"]
    if not args.no_cpu_baseline:
        print("[bench] timing the CPU oracle baseline", file=sys.stderr, flush=True)
        record["cpu_baseline"] = cpu_baseline(metadata, caches[0], q, k, v, ctx, args.cpu_budget)
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
