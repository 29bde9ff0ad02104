"""GPU: repeated launches give bit-identical results.

Every kernel here assigns each output row, partial slot and pool slot to
exactly one wave, so a step run again must reproduce its outputs bit for bit.
A race (two waves on one row), a read of memory nothing wrote in this launch
(a stale split-K partial) or a missing wait would show up as a difference
between runs.  Each step runs three times on one backend; between the runs a
different step on the same backend overwrites the shared split-K workspace
with other partials.  Outputs of the first run are also checked against the
oracle, and the pool slots the step appends are compared after every run.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import light_vllm_amd as lv
from paged_cases import make_step, oracle_attention, tolerances

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)


def _tree(rng, n):
    parents = [-1] + [int(rng.integers(0, i)) for i in range(1, n - 1)]
    return tuple([-1] + [0 if p == -1 else p + 1 for p in parents])


def _decode_step(dtype, seed):
    rng = np.random.default_rng(seed)
    computed = [int(c) for c in rng.integers(200, 3000, size=16)]
    return make_step(hq=28, hkv=4, d=128, bs=16, dtype=dtype, computed=computed, layouts=[(-1,)] * 16, seed=seed)


def _tree_step(seed):
    # Eight draft trees over a shared 2,048-token prefix: split-K prefill
    # with shared-prefix spans, and the merge of both kinds of partials.
    rng = np.random.default_rng(seed)
    computed = [2048 + int(s) for s in rng.integers(64, 513, size=8)]
    return make_step(hq=12, hkv=2, d=128, bs=16, dtype=torch.bfloat16, computed=computed,
                     layouts=[_tree(rng, 9) for _ in range(8)], shared_prefix_blocks=128, seed=seed)


def _mixed_step(seed):
    # Two prompt chunks and decode rows in one step (prefill + decode kernels).
    rng = np.random.default_rng(seed)
    computed = [int(c) for c in rng.integers(0, 2000, size=2)] + [int(c) for c in rng.integers(256, 3000, size=6)]
    layouts = [tuple(range(-1, n - 1)) for n in (300, 177)] + [(-1,)] * 6
    return make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=computed, layouts=layouts,
                     seed=seed)


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int32 if t.element_size() == 4 else torch.int16)


def _run(backend, step):
    lid = step.layer_ids[0]
    ctx = backend.create(step.cache, step.metadata)
    out = ctx.forward(lid, step.query, step.key, step.value, scale=step.scale)
    torch.cuda.synchronize()
    slots = step.metadata.slot_mapping(block_size=step.cache.config.block_size, device=step.query.device)
    layer = step.cache.layer(lid)
    nslots = step.cache.config.num_blocks * step.cache.config.block_size
    hkv, d = step.key.shape[1:]
    assert torch.equal(layer.keys.view(nslots, hkv, d).index_select(0, slots), step.key)
    assert torch.equal(layer.values.view(nslots, hkv, d).index_select(0, slots), step.value)
    return out.clone()


def _short_decode_step(seed):
    # Short contexts: the workgroup split (eight waves per segment, LDS merge).
    rng = np.random.default_rng(seed)
    computed = [int(c) for c in rng.integers(0, 370, size=16)]
    return make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=computed, layouts=[(-1,)] * 16,
                     seed=seed)


CASES = {
    "short decode (workgroup split)": lambda: _short_decode_step(67),
    "decode bf16": lambda: _decode_step(torch.bfloat16, 61),
    "decode fp32": lambda: _decode_step(torch.float32, 62),
    "trees over a shared prefix": lambda: _tree_step(63),
    "chunks and decode rows": lambda: _mixed_step(64),
}


@pytest.mark.parametrize("waves", (4, 8))
@pytest.mark.parametrize("name", sorted(CASES))
def test_repeated_steps_are_bit_identical(name, waves) -> None:
    print(f"[gpu] repeat {name} waves={waves}", file=sys.stderr, flush=True)
    step = CASES[name]()
    other = _tree_step(65) if "tree" not in name else _decode_step(torch.bfloat16, 66)
    backend = lv.HipPagedAttentionBackend(prefill_waves=waves)
    first = _run(backend, step)
    expect = oracle_attention(step, step.layer_ids[0])
    err = np.abs(first.float().cpu().numpy() - expect)
    max_tol, mean_tol = tolerances(step.query.dtype)
    assert err.max() <= max_tol and err.mean() <= mean_tol, (err.max(), err.mean())
    for _ in range(2):
        _run(backend, other)  # other partials into the shared workspace
        again = _run(backend, step)
        assert torch.equal(_bits(again), _bits(first))
