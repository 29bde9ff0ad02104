"""Randomised GPU parity: whole model steps drawn at random.

Each seed draws a head geometry, dtype, block size (seeds 64-79: 3 or 12,
the kernels' path for block sizes that are not powers of two) and a batch
mixing decode tokens, causal chunks, draft trees, lookahead reservations and an optional
shared read-only prefix, then runs forward (optionally with RoPE fused into
the append, and with either prefill workgroup shape) and checks the result
against the CPU oracle at the dtype's tolerance (bf16 2e-2 / 2e-3, fp16
3e-3 / 3e-4, fp32 1e-5 max-abs / 1e-6 mean-abs), plus the step's K/V rows bit
for bit at their slots.  The draws stay small enough for the per-query
oracle.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import light_vllm_amd as lv
from oracle import paged_kv_oracle as O
from paged_cases import DTYPES, make_step, oracle_attention, tolerances

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

DEV = torch.device("cuda:0")
NAMES = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}
GEOMETRIES = [(28, 4, 128), (12, 2, 128), (14, 2, 64), (8, 8, 64), (16, 2, 80), (16, 4, 96), (8, 2, 256),
              (32, 4, 32), (12, 4, 48), (16, 2, 112), (8, 2, 160), (16, 4, 192), (4, 2, 240)]


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    return t.numpy().copy() if t.dtype == torch.float32 else t.view(torch.int16).numpy().view(np.uint16).copy()


def _rope(positions, d, dtype):
    pos = torch.as_tensor(np.asarray(positions), dtype=torch.float32)
    freqs = 1.0 / (1_000_000.0 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    emb = torch.outer(pos, freqs)
    emb = torch.cat((emb, emb), dim=-1)
    return emb.cos().to(dtype).to(DEV), emb.sin().to(dtype).to(DEV)


def _draw(seed: int):
    rng = np.random.default_rng(seed)
    hq, hkv, d = GEOMETRIES[int(rng.integers(len(GEOMETRIES)))]
    dtype = DTYPES[str(rng.choice(["bf16", "bf16", "fp16", "fp32"]))]
    if d == 32 and dtype != torch.float32:
        dtype = torch.bfloat16
    bs = int(rng.choice([1, 4, 16, 16, 32]))
    if seed >= 64:  # block sizes that are not powers of two (the kernels' division path)
        bs = (3, 12)[seed % 2]
    batch = int(rng.integers(1, 7))
    shared = int(rng.integers(0, 3)) * max(1, 64 // bs)  # shared read-only prefix blocks
    computed, layouts, reserved = [], [], []
    for _ in range(batch):
        kind = rng.choice(["decode", "decode", "chunk", "tree"])
        c = shared * bs + int(rng.integers(0, 700))
        if kind == "decode":
            q = (-1,)
        elif kind == "chunk":
            q = tuple(range(-1, int(rng.integers(2, 90)) - 1))
        else:
            n = int(rng.integers(2, 12))
            q = tuple([-1] + [int(rng.integers(0, i)) for i in range(1, n)])
        computed.append(c)
        layouts.append(q)
        reserved.append(len(q) + int(rng.integers(0, 3)))  # lookahead slots
    opts = dict(rotary=bool(rng.integers(0, 2)), waves=int(rng.choice([4, 8])),
                prefill=bool(rng.integers(0, 4)))  # mostly with the prefill kernel
    return dict(hq=hq, hkv=hkv, d=d, bs=bs, dtype=dtype, computed=computed, layouts=layouts, reserved=reserved,
                shared_prefix_blocks=shared, seed=seed), opts


@pytest.mark.parametrize("seed", range(80))
def test_random_step_matches_the_oracle(seed) -> None:
    case, opts = _draw(seed)
    print(f"[gpu] random step seed {seed}: {case['hq']}/{case['hkv']}x{case['d']} {case['dtype']} bs {case['bs']} "
          f"q_lens {[len(l) for l in case['layouts']]} {opts}", file=sys.stderr, flush=True)
    step = make_step(**case)
    lid = step.layer_ids[0]
    backend = lv.HipPagedAttentionBackend(use_prefill_kernel=opts["prefill"], prefill_waves=opts["waves"])
    ctx = backend.create(step.cache, step.metadata)
    dtype = case["dtype"]
    key_rows, query = _bits(step.key), None
    if opts["rotary"]:
        positions = [p for c, l in zip(step.metadata.num_computed_tokens, step.metadata.query_layouts)
                     for p in O.semantic_positions(tuple(l.parent_indices), c)]
        cos, sin = _rope(positions, case["d"], dtype)
        q_rot = O.rotary_half(_bits(step.query), _bits(cos), _bits(sin), NAMES[dtype])
        key_rows = O.rotary_half(_bits(step.key), _bits(cos), _bits(sin), NAMES[dtype])
        query = torch.from_numpy(q_rot if dtype == torch.float32 else q_rot.view(np.int16))
        query = query if dtype == torch.float32 else query.view(dtype)
        out = ctx.forward(lid, step.query, step.key, step.value, scale=step.scale, rotary=(cos, sin))
    else:
        out = ctx.forward(lid, step.query, step.key, step.value, scale=step.scale)
    torch.cuda.synchronize()
    cfg = step.cache.config
    slots = step.metadata.slot_mapping(block_size=cfg.block_size, device=DEV)
    layer = step.cache.layer(lid)
    n = cfg.num_blocks * cfg.block_size
    hkv, d = step.key.shape[1:]
    np.testing.assert_array_equal(_bits(layer.keys.view(n, hkv, d).index_select(0, slots)), key_rows)
    np.testing.assert_array_equal(_bits(layer.values.view(n, hkv, d).index_select(0, slots)), _bits(step.value))
    expect = oracle_attention(step, lid, query=query)
    got = out.float().cpu().numpy()
    err = np.abs(got - expect)
    max_tol, mean_tol = tolerances(dtype)
    assert np.isfinite(got).all()
    assert err.max() <= max_tol, f"max-abs {err.max():.3e} > {max_tol}"
    assert err.mean() <= mean_tol, f"mean-abs {err.mean():.3e} > {mean_tol}"
