"""GPU: whole model steps at the BASELINE shapes, not one layer at a time.

* C4: one ``create()`` over a 28-layer cache of 16 x 32K contexts (28 pools,
  30 GB), the step's 28 ``forward`` calls, then layers 0, 9, 18 and 27
  checked against the fp64 dense oracle with their appended K/V bit for bit.
* C5: the speculative step as light-vllm runs it, over two layers: the
  copy-on-write of the last shared prefix page into each sequence's private
  page (pools byte-compared with the oracle's block copy), tree verification
  of 32 draft trees over the 2,048-token shared prefix (outputs against the
  oracle, appended K/V bit for bit), then ``compact_many`` of the accepted
  paths (pools byte-compared with the oracle's compact, moved counts equal).
"""

from __future__ import annotations

import math
import sys

import numpy as np
import pytest
import torch

import light_vllm_amd as lv
from oracle import paged_kv_oracle as O
from paged_cases import Step, dense_oracle_attention, oracle_attention, report_margin, tolerances

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

DEV = torch.device("cuda:0")


def _announce(name: str) -> None:
    print(f"[gpu] {name}", file=sys.stderr, flush=True)


def _fill(cache, layer_ids, seed: int) -> None:
    gen = torch.Generator(device=DEV).manual_seed(seed)
    for lid in layer_ids:
        for pool in (cache.layer(lid).keys, cache.layer(lid).values):
            pool.copy_(torch.randn(pool.shape, generator=gen, device=DEV, dtype=torch.float32).to(pool.dtype))


def _check_appended(step: Step, lid: str, key, value) -> None:
    slots = step.metadata.slot_mapping(block_size=step.cache.config.block_size, device=DEV)
    layer = step.cache.layer(lid)
    nslots = step.cache.config.num_blocks * step.cache.config.block_size
    hkv, d = key.shape[1:]
    assert torch.equal(layer.keys.view(nslots, hkv, d).index_select(0, slots), key)
    assert torch.equal(layer.values.view(nslots, hkv, d).index_select(0, slots), value)


# ------------------------------------------------------------------ C4
C4_LAYERS = 28
C4_CHECKED = (0, 9, 18, 27)


@pytest.fixture(scope="module")
def c4_step():
    _announce("C4 whole step: 28 layers, 16 x 32768")
    hq, hkv, d, bs, batch, ctx = 28, 4, 128, 16, 16, 32768
    per_seq = (ctx + 1 + bs - 1) // bs
    num_blocks = batch * per_seq + 16
    rng = np.random.default_rng(4404)
    perm = [int(b) for b in rng.permutation(num_blocks)]
    tables = tuple(tuple(perm[r * per_seq : (r + 1) * per_seq]) for r in range(batch))
    md = lv.PagedAttentionMetadata(block_tables=tables, num_computed_tokens=(ctx,) * batch,
                                   query_layouts=tuple(lv.linear_query_layout(1) for _ in range(batch)))
    layer_ids = tuple(f"layer{i}" for i in range(C4_LAYERS))
    spec = lv.ModelKVCacheSpec(tuple(lv.AttentionLayerSpec(lid, hq, hkv, d) for lid in layer_ids))
    cache = lv.PagedKVCache(spec, lv.PagedKVCacheConfig(num_blocks=num_blocks, block_size=bs,
                                                        dtype=torch.bfloat16, device=DEV))
    _fill(cache, layer_ids, 4404)
    gen = torch.Generator(device=DEV).manual_seed(4405)
    inputs = [tuple(torch.randn((batch, h, d), generator=gen, device=DEV).to(torch.bfloat16) for h in (hq, hkv, hkv))
              for _ in layer_ids]
    ctx_obj = lv.HipPagedAttentionBackend().create(cache, md)
    outs = [ctx_obj.forward(lid, *inputs[i], scale=1.0 / math.sqrt(d)) for i, lid in enumerate(layer_ids)]
    torch.cuda.synchronize()
    assert ctx_obj.layer_ids == frozenset(layer_ids)
    work = ctx_obj.work_of(spec.layers[0])
    assert work.num_jobs == batch  # every 32K row split over waves and merged
    yield cache, md, layer_ids, inputs, outs, 1.0 / math.sqrt(d)
    del cache, outs
    torch.cuda.empty_cache()


@pytest.mark.parametrize("index", C4_CHECKED)
def test_c4_whole_step_layer_matches_the_dense_oracle(c4_step, index) -> None:
    cache, md, layer_ids, inputs, outs, scale = c4_step
    lid = layer_ids[index]
    _announce(f"C4 whole step: check {lid}")
    q, k, v = inputs[index]
    step = Step(cache, md, q, k, v, layer_ids, scale)
    _check_appended(step, lid, k, v)
    got = outs[index].float().cpu().numpy()
    err = np.abs(got - dense_oracle_attention(step, lid))
    max_tol, mean_tol = tolerances(torch.bfloat16)
    report_margin(f"C4 whole step {lid}", err, torch.bfloat16)
    assert np.isfinite(got).all()
    assert err.max() <= max_tol and err.mean() <= mean_tol, (lid, err.max(), err.mean())


# ------------------------------------------------------------------ C5
def _bits(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.int16).cpu().numpy().copy()


def test_c5_whole_step_copy_verify_compact() -> None:
    _announce("C5 whole step: COW, tree verification over 2 layers, compact_many")
    hq, hkv, d, bs, batch, prefix, tree = 12, 2, 128, 16, 32, 2048, 8
    rng = np.random.default_rng(5505)
    shared_blocks = prefix // bs
    suffix = [int(s) for s in rng.integers(64, 513, size=batch)]
    computed = [prefix + s for s in suffix]
    q_len = 1 + tree
    layouts, accepted = [], []
    for _ in range(batch):
        parents = [-1] + [int(rng.integers(0, i)) for i in range(1, tree)]
        layouts.append(tuple([-1] + [0 if p == -1 else p + 1 for p in parents]))
        leaf = int(rng.integers(0, tree))
        path = [leaf]
        while parents[path[-1]] != -1:
            path.append(parents[path[-1]])
        accepted.append((0,) + tuple(sorted(i + 1 for i in path)))
    need = [(c + q_len + bs - 1) // bs for c in computed]
    num_blocks = shared_blocks + sum(n - shared_blocks + 1 for n in need) + 16
    perm = [int(b) for b in rng.permutation(num_blocks)]
    shared, free = perm[:shared_blocks], perm[shared_blocks:]
    tables, cow_dst, off = [], [], 0
    for n in need:
        # The last shared page is copied on write into a private page.
        private = free[off : off + n - shared_blocks + 1]
        off += n - shared_blocks + 1
        cow_dst.append(private[0])
        tables.append(tuple(shared[:-1]) + tuple(private))
    cow_src = [shared[-1]] * batch
    md = lv.PagedAttentionMetadata(block_tables=tuple(tables), num_computed_tokens=tuple(computed),
                                   query_layouts=tuple(lv.QueryLayout(p) for p in layouts),
                                   num_readonly_prefix_blocks=(shared_blocks - 1,) * batch)
    layer_ids = ("layer0", "layer1")
    spec = lv.ModelKVCacheSpec(tuple(lv.AttentionLayerSpec(lid, hq, hkv, d) for lid in layer_ids))
    cache = lv.PagedKVCache(spec, lv.PagedKVCacheConfig(num_blocks=num_blocks, block_size=bs,
                                                        dtype=torch.bfloat16, device=DEV))
    _fill(cache, layer_ids, 5505)
    pools = [(_bits(cache.layer(lid).keys), _bits(cache.layer(lid).values)) for lid in layer_ids]

    # 1. Copy-on-write of the partial prefix page, every layer, K and V.
    cache.copy_blocks(cow_src, cow_dst)
    torch.cuda.synchronize()
    O.block_copy(pools, cow_src, cow_dst)
    for lid, (kb, vb) in zip(layer_ids, pools):
        np.testing.assert_array_equal(_bits(cache.layer(lid).keys), kb)
        np.testing.assert_array_equal(_bits(cache.layer(lid).values), vb)

    # 2. Tree verification, one context for the step, each layer its own Q/K/V.
    gen = torch.Generator(device=DEV).manual_seed(5506)
    t = batch * q_len
    ctx = lv.HipPagedAttentionBackend().create(cache, md)
    assert ctx.work_of(spec.layers[0]).num_prefill_units > 0
    max_tol, mean_tol = tolerances(torch.bfloat16)
    scale = 1.0 / math.sqrt(d)
    for lid in layer_ids:
        q, k, v = (torch.randn((t, h, d), generator=gen, device=DEV).to(torch.bfloat16) for h in (hq, hkv, hkv))
        out = ctx.forward(lid, q, k, v, scale=scale)
        torch.cuda.synchronize()
        step = Step(cache, md, q, k, v, layer_ids, scale)
        _check_appended(step, lid, k, v)
        err = np.abs(out.float().cpu().numpy() - oracle_attention(step, lid))
        report_margin(f"C5 whole step {lid}", err, torch.bfloat16)
        assert err.max() <= max_tol and err.mean() <= mean_tol, (lid, err.max(), err.mean())
    assert ctx.layer_ids == frozenset(layer_ids)

    # 3. Compact every request's accepted path in one launch.
    pools = [(_bits(cache.layer(lid).keys), _bits(cache.layer(lid).values)) for lid in layer_ids]
    requests, expect = [], []
    for r in range(batch):
        args = dict(num_computed_tokens=computed[r], num_query_tokens=q_len, num_reserved_query_tokens=q_len,
                    retained_query_indices=accepted[r], num_readonly_prefix_blocks=shared_blocks - 1)
        expect.append(O.compact(pools, tables[r], num_blocks=num_blocks, block_size=bs, **args))
        requests.append(dict(block_ids=tables[r], **args))
    moved = cache.compact_many(requests)
    torch.cuda.synchronize()
    assert moved == tuple(expect) and sum(moved) > 0
    for lid, (kb, vb) in zip(layer_ids, pools):
        np.testing.assert_array_equal(_bits(cache.layer(lid).keys), kb)
        np.testing.assert_array_equal(_bits(cache.layer(lid).values), vb)
