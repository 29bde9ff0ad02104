"""GPU: the copy-on-write producer end to end.

New sequences start from a donor's first P tokens (P inside a page):
``share_prefix`` gives their tables and copy commands, ``copy_blocks``
copies the donor's partial page into each private page on the GPU (checked
byte for byte against the oracle's block_copy closed form over the whole
pools, every layer, K and V), and a tree-verify step over the new tables
(the shared readonly pages, the copied page, private pages) matches the
oracle's attention, the donor's decode row included.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import light_vllm_amd as lv
from oracle import paged_kv_oracle as O
from paged_cases import DTYPES, Step, oracle_attention, tolerances

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

DEV = torch.device("cuda:0")


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy().copy()


@pytest.mark.parametrize("bs,shared", ((16, 2040), (16, 200), (12, 777), (3, 50)))
@pytest.mark.parametrize("dtype", ("bf16", "fp16"))
def test_copied_starts_verify_trees_against_the_oracle(bs, shared, dtype) -> None:
    print(f"[gpu] prefix COW bs={bs} shared={shared} {dtype}", file=sys.stderr, flush=True)
    rng = np.random.default_rng(bs * 1000 + shared)
    hq, hkv, d, layers = 12, 2, 128, 2
    torch_dtype = DTYPES[dtype]
    donor_computed = shared + 37
    donor = tuple(int(b) for b in rng.permutation(4096)[: -(-(donor_computed + 1) // bs)])
    free = [int(b) for b in rng.permutation(4096) if int(b) not in set(donor)]
    readonly = shared // bs
    starts = [lv.share_prefix(donor, readonly, shared, block_size=bs, allocate_block=free.pop) for _ in range(5)]
    tables, computed, layouts = [donor], [donor_computed], [(-1,)]
    for s in starts:
        parents = tuple([-1] + [int(rng.integers(0, i)) for i in range(1, 9)])
        need = -(-(s.num_computed_tokens + len(parents)) // bs)
        tables.append(s.block_ids + tuple(free.pop() for _ in range(need - len(s.block_ids))))
        computed.append(s.num_computed_tokens)
        layouts.append(parents)
    md = lv.PagedAttentionMetadata(
        block_tables=tuple(tables), num_computed_tokens=tuple(computed),
        query_layouts=tuple(lv.QueryLayout(p) for p in layouts),
        num_readonly_prefix_blocks=(readonly,) + tuple(s.num_readonly_prefix_blocks for s in starts))
    layer_ids = tuple(f"layer{i}" for i in range(layers))
    spec = lv.ModelKVCacheSpec(tuple(lv.AttentionLayerSpec(i, hq, hkv, d) for i in layer_ids))
    cache = lv.PagedKVCache(spec, lv.PagedKVCacheConfig(num_blocks=4096, block_size=bs, dtype=torch_dtype,
                                                        device=DEV))
    gen = torch.Generator(device="cpu").manual_seed(bs + shared)
    for lid in layer_ids:  # every page random: the copy must move exactly the partial pages
        for pool in (cache.layer(lid).keys, cache.layer(lid).values):
            pool.copy_(torch.randn(pool.shape, generator=gen).to(torch_dtype))
    before = {lid: (_bits(cache.layer(lid).keys), _bits(cache.layer(lid).values)) for lid in layer_ids}
    src, dst = lv.copy_commands(starts)
    assert len(src) == (len(starts) if shared % bs else 0)
    cache.copy_blocks(src, dst)
    torch.cuda.synchronize()
    for lid in layer_ids:
        kp, vp = before[lid]
        O.block_copy([(kp, vp)], src, dst)
        assert np.array_equal(_bits(cache.layer(lid).keys), kp)
        assert np.array_equal(_bits(cache.layer(lid).values), vp)
    t = sum(len(p) for p in layouts)
    q = torch.randn((t, hq, d), generator=gen).to(torch_dtype).to(DEV)
    k = torch.randn((t, hkv, d), generator=gen).to(torch_dtype).to(DEV)
    v = torch.randn((t, hkv, d), generator=gen).to(torch_dtype).to(DEV)
    step = Step(cache, md, q, k, v, layer_ids, 1.0 / np.sqrt(d))
    ctx = lv.HipPagedAttentionBackend().create(cache, md)
    max_tol, mean_tol = tolerances(torch_dtype)
    for lid in layer_ids:
        out = ctx.forward(lid, q, k, v, scale=step.scale)
        torch.cuda.synchronize()
        expect = oracle_attention(step, lid)
        err = np.abs(out.float().cpu().numpy() - expect)
        assert err.max() <= max_tol and err.mean() <= mean_tol, (err.max(), err.mean())
