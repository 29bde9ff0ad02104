"""GPU parity at the BASELINE configurations' full sizes (one layer each).

C2 at full size is in test_gpu_attention.py.  These cover C3 (8 chunks of 512
with prior context plus 56 decode tokens), C4 (16 x 32K contexts, one layer of
the 28, 1 GiB pool) and C5 (32 sequences sharing a 2048-token prefix, 9-token
trees), each checked against the independent fp64 dense oracle with the bf16
tolerances of paged_cases.tolerances, plus the bit-exact pool state of the
step's K/V.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from paged_cases import dense_oracle_attention, make_step, report_margin, tolerances

import light_vllm_amd as lv

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

DEV = torch.device("cuda:0")


def _announce(name: str) -> None:
    print(f"[gpu] {name}", file=sys.stderr, flush=True)


def _lin(*lengths):
    return [tuple(range(-1, n - 1)) for n in lengths]


def _run(step, margin: str):
    ctx = lv.HipPagedAttentionBackend().create(step.cache, step.metadata)
    lid = step.layer_ids[0]
    out = ctx.forward(lid, step.query, step.key, step.value, scale=step.scale)
    torch.cuda.synchronize()
    slots = step.metadata.slot_mapping(block_size=step.cache.config.block_size, device=DEV)
    layer = step.cache.layer(lid)
    nslots = step.cache.config.num_blocks * step.cache.config.block_size
    hkv, d = step.key.shape[1:]
    assert torch.equal(layer.keys.view(nslots, hkv, d).index_select(0, slots), step.key)
    assert torch.equal(layer.values.view(nslots, hkv, d).index_select(0, slots), step.value)
    got = out.float().cpu().numpy()
    err = np.abs(got - dense_oracle_attention(step, lid))
    max_tol, mean_tol = tolerances(step.query.dtype)
    report_margin(margin, err, step.query.dtype)
    assert np.isfinite(got).all()
    assert err.max() <= max_tol, f"max-abs {err.max():.3e} > {max_tol}"
    assert err.mean() <= mean_tol, f"mean-abs {err.mean():.3e} > {mean_tol}"
    return ctx


def test_c3_full_mixed_batch() -> None:
    _announce("C3 full: 8 x 512 prefill + 56 decode")
    rng = np.random.default_rng(3003)
    computed = [int(c) for c in rng.integers(0, 3073, size=8)] + [int(c) for c in rng.integers(256, 4097, size=56)]
    step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=computed,
                     layouts=_lin(*([512] * 8 + [1] * 56)), seed=3003)
    ctx = _run(step, "C3 (bf16, prefill + decode rows)")
    work = ctx.work_of(step.cache.layer_spec(step.layer_ids[0]))
    assert work.num_prefill_units > 0 and work.waves_per_head > 0


def test_c4_full_one_layer_32k_contexts() -> None:
    _announce("C4 full: 16 x 32768, one layer")
    step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=[32768] * 16,
                     layouts=_lin(*([1] * 16)), num_blocks=32800, seed=4004)
    ctx = _run(step, "C4 (bf16, stream-K, 16 partials per row)")
    work = ctx.work_of(step.cache.layer_spec(step.layer_ids[0]))
    assert work.num_jobs == 16  # every 32K sequence is split across waves and merged


def test_c5_full_tree_verification_shared_prefix() -> None:
    _announce("C5 full: 32 trees over a shared 2048-token prefix")
    rng = np.random.default_rng(5005)
    layouts, computed = [], []
    for _ in range(32):
        parents = [-1] + [int(rng.integers(0, i)) for i in range(1, 8)]
        layouts.append(tuple([-1] + [0 if p == -1 else p + 1 for p in parents]))
        computed.append(2048 + int(rng.integers(64, 513)))
    step = make_step(hq=12, hkv=2, d=128, bs=16, dtype=torch.bfloat16, computed=computed, layouts=layouts,
                     shared_prefix_blocks=128, seed=5005)
    ctx = _run(step, "C5 (bf16, split-K prefill + spans)")
    work = ctx.work_of(step.cache.layer_spec(step.layer_ids[0]))
    assert work.num_prefill_partial_slots > 0  # split-K tree verification
