"""Seeded paged-KV test cases shared by the GPU parity tests.

A case is one model step: a pool whose history positions hold N(0,1) values,
block tables drawn from a random permutation of the pool (disjoint except an
optional shared read-only prefix), and this step's Q/K/V.  History is written
with plain torch indexing (test setup, independent of the kernels under test).
"""

from __future__ import annotations

import math
import sys
from dataclasses import dataclass

import numpy as np
import torch

import light_vllm_amd as lv
from oracle import paged_kv_oracle as O

DTYPES = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


@dataclass
class Step:
    cache: lv.PagedKVCache
    metadata: lv.PagedAttentionMetadata
    query: torch.Tensor
    key: torch.Tensor
    value: torch.Tensor
    layer_ids: tuple[str, ...]
    scale: float


def make_step(
    *,
    hq: int,
    hkv: int,
    d: int,
    bs: int,
    dtype: torch.dtype,
    computed,
    layouts,
    seed: int,
    num_blocks: int | None = None,
    reserved=None,
    shared_prefix_blocks: int = 0,
    num_layers: int = 1,
    device: str = "cuda:0",
    prefix_groups=None,
    group_prefix_blocks=(),
) -> Step:
    """A step of requests with random history.  Every request shares the first
    ``shared_prefix_blocks`` blocks (readonly); or, with ``prefix_groups`` (per
    request: an index into ``group_prefix_blocks``, or -1), each group of
    requests shares its own readonly prefix of that many blocks."""
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device="cpu").manual_seed(seed)
    computed = [int(c) for c in computed]
    layouts = [lv.QueryLayout(tuple(p)) if not isinstance(p, lv.QueryLayout) else p for p in layouts]
    q_lens = [len(l) for l in layouts]
    reserved = [int(r) for r in (reserved or q_lens)]
    need = [(c + r + bs - 1) // bs for c, r in zip(computed, reserved)]
    if prefix_groups is None:
        prefix_groups = [0] * len(need)
        group_prefix_blocks = (shared_prefix_blocks,)
    own = [len(group_prefix_blocks) and group_prefix_blocks[g] if g >= 0 else 0 for g in prefix_groups]
    total = sum(group_prefix_blocks) + sum(n - o for n, o in zip(need, own))
    nb = num_blocks or total + 7
    assert nb >= total
    perm = [int(x) for x in rng.permutation(nb)]
    prefixes, off = [], 0
    for blocks in group_prefix_blocks:
        prefixes.append(perm[off : off + blocks])
        off += blocks
    rest = perm[off:]
    tables = []
    for n, g in zip(need, prefix_groups):
        shared = prefixes[g] if g >= 0 else []
        tables.append(tuple(shared + rest[: n - len(shared)]))
        rest = rest[n - len(shared) :]
    readonly = tuple(group_prefix_blocks[g] if g >= 0 else 0 for g in prefix_groups)
    layer_ids = tuple(f"layer{i}" for i in range(num_layers))
    spec = lv.ModelKVCacheSpec(tuple(lv.AttentionLayerSpec(i, hq, hkv, d) for i in layer_ids))
    cache = lv.PagedKVCache(spec, lv.PagedKVCacheConfig(num_blocks=nb, block_size=bs, dtype=dtype, device=device))
    # History: every position < computed of every request (shared prefix written once).
    hist_slots = []
    for table, c in zip(tables, computed):
        for pos in range(c):
            hist_slots.append(table[pos // bs] * bs + pos % bs)
    hist = torch.tensor(sorted(set(hist_slots)), dtype=torch.long)
    for lid in layer_ids:
        layer = cache.layer(lid)
        for pool in (layer.keys, layer.values):
            flat = pool.view(nb * bs, hkv, d)
            if hist.numel():
                vals = torch.randn((hist.numel(), hkv, d), generator=gen, dtype=torch.float32).to(dtype)
                flat[hist.to(device)] = vals.to(device)
    t = sum(q_lens)
    query = torch.randn((t, hq, d), generator=gen, dtype=torch.float32).to(dtype).to(device)
    key = torch.randn((t, hkv, d), generator=gen, dtype=torch.float32).to(dtype).to(device)
    value = torch.randn((t, hkv, d), generator=gen, dtype=torch.float32).to(dtype).to(device)
    metadata = lv.PagedAttentionMetadata(
        block_tables=tuple(tables),
        num_computed_tokens=tuple(computed),
        query_layouts=tuple(layouts),
        num_reserved_query_tokens=tuple(reserved),
        num_readonly_prefix_blocks=readonly if any(readonly) else (),
    )
    return Step(cache, metadata, query, key, value, layer_ids, 1.0 / math.sqrt(d))


def referenced_pool(cache, layer_id: str, metadata) -> tuple[np.ndarray, np.ndarray, list[tuple[int, ...]]]:
    """fp32 copies of only the blocks the tables reference, with remapped tables."""

    used = sorted({b for table in metadata.block_tables for b in table})
    index = {b: i for i, b in enumerate(used)}
    idx = torch.tensor(used, dtype=torch.long, device=cache.config.device)
    layer = cache.layer(layer_id)
    k = layer.keys.index_select(0, idx).float().cpu().numpy()
    v = layer.values.index_select(0, idx).float().cpu().numpy()
    tables = [tuple(index[b] for b in table) for table in metadata.block_tables]
    return k, v, tables


def oracle_attention(step: Step, layer_id: str, query: torch.Tensor | None = None) -> np.ndarray:
    """Oracle output for the pool as it is now (after this step's append)."""

    k, v, tables = referenced_pool(step.cache, layer_id, step.metadata)
    q = (step.query if query is None else query).float().cpu().numpy()
    parents = [l.parent_indices for l in step.metadata.query_layouts]
    return O.paged_attention(q, k, v, tables, step.metadata.num_computed_tokens, parents, scale=step.scale)


def dense_oracle_attention(step: Step, layer_id: str) -> np.ndarray:
    """Independent fp64 masked-softmax oracle (vectorised per request), for
    steps too large for the per-query online-softmax restatement."""

    k, v, tables = referenced_pool(step.cache, layer_id, step.metadata)
    q = step.query.float().cpu().numpy()
    parents = [l.parent_indices for l in step.metadata.query_layouts]
    return O.dense_attention(q, k, v, tables, step.metadata.num_computed_tokens, parents, scale=step.scale)


def report_margin(config: str, err: np.ndarray, dtype: torch.dtype) -> None:
    """Print a ``[margin]`` line: the errors against the tolerances, as a
    share of each (the numerical margin table is built from these lines)."""

    max_tol, mean_tol = tolerances(dtype)
    mx, mean = float(err.max()), float(err.mean())
    print(f"[margin] {config}: max-abs {mx:.3e} ({100 * mx / max_tol:.1f}% of {max_tol:g}), "
          f"mean-abs {mean:.3e} ({100 * mean / mean_tol:.1f}% of {mean_tol:g})", file=sys.stderr, flush=True)


def tolerances(dtype: torch.dtype) -> tuple[float, float]:
    """(max-abs, mean-abs) bounds: bf16 2e-2 / 2e-3 and fp32 1e-5 (the target's),
    fp16 3e-3 (the reference Triton test's fp16 atol) / 3e-4."""

    if dtype == torch.bfloat16:
        return 2e-2, 2e-3
    if dtype == torch.float16:
        return 3e-3, 3e-4
    return 1e-5, 1e-6
