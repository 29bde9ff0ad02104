"""GPU parity of the MFMA chunked-prefill kernel against the CPU oracle.

Requests whose queries x group exceed one 16-column MFMA tile take the
prefill kernel in a bf16/fp16 layer; the others take the decode kernel in the
same step.  When there are fewer prefill units than resident workgroups the
planner splits their key ranges (split-K) and a merge combines the partials.  Tolerances as in
paged_cases.tolerances (bf16 max-abs 2e-2 / mean-abs 2e-3, fp16 3e-3 / 3e-4).
Large steps are checked against the independent fp64 dense oracle.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import light_vllm_amd as lv
from paged_cases import DTYPES, dense_oracle_attention, make_step, oracle_attention, tolerances

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

DEV = torch.device("cuda:0")


def _announce(name: str) -> None:
    print(f"[gpu] {name}", file=sys.stderr, flush=True)


def _lin(*lengths):
    return [tuple(range(-1, n - 1)) for n in lengths]


WAVES = (4, 8)  # both prefill workgroup shapes (8 falls back to 4 at head size 256)


def _check(step, *, backend=None, dense=False, expect_prefill=True, waves=None):
    backend = backend or lv.HipPagedAttentionBackend(prefill_waves=waves)
    ctx = backend.create(step.cache, step.metadata)
    lid = step.layer_ids[0]
    out = ctx.forward(lid, step.query, step.key, step.value, scale=step.scale)
    torch.cuda.synchronize()
    spec = step.cache.layer_spec(lid)
    work = ctx.work_of(spec)
    assert (work.num_prefill_units > 0) == expect_prefill
    if waves is not None and expect_prefill:
        assert work.prefill_waves == (waves if spec.head_size <= 128 else 4)
    slots = step.metadata.slot_mapping(block_size=step.cache.config.block_size, device=DEV)
    layer = step.cache.layer(lid)
    nslots = step.cache.config.num_blocks * step.cache.config.block_size
    hkv, d = step.key.shape[1:]
    assert torch.equal(layer.keys.view(nslots, hkv, d).index_select(0, slots), step.key)
    assert torch.equal(layer.values.view(nslots, hkv, d).index_select(0, slots), step.value)
    expect = dense_oracle_attention(step, lid) if dense else oracle_attention(step, lid)
    got = out.float().cpu().numpy()
    err = np.abs(got - expect)
    max_tol, mean_tol = tolerances(step.query.dtype)
    assert np.isfinite(got).all()
    assert err.max() <= max_tol, f"max-abs {err.max():.3e} > {max_tol}"
    assert err.mean() <= mean_tol, f"mean-abs {err.mean():.3e} > {mean_tol}"
    return out


@pytest.mark.parametrize("waves", WAVES)
@pytest.mark.parametrize("dtype", ("bf16", "fp16"))
@pytest.mark.parametrize("head_size", range(32, 257, 16))
def test_prefill_head_sizes_and_dtypes(dtype, head_size, waves) -> None:
    _announce(f"prefill d={head_size} {dtype} waves={waves}")
    step = make_step(hq=8, hkv=2, d=head_size, bs=16, dtype=DTYPES[dtype], computed=[0, 37, 300, 90],
                     layouts=_lin(40, 100, 17, 1), seed=head_size + 7)
    _check(step, waves=waves)


@pytest.mark.parametrize("waves", WAVES)
@pytest.mark.parametrize("bs", (1, 3, 16, 32))
def test_prefill_block_sizes(bs, waves) -> None:
    _announce(f"prefill block size {bs} waves={waves}")
    step = make_step(hq=28, hkv=4, d=128, bs=bs, dtype=torch.bfloat16, computed=[5, 140, 0],
                     layouts=_lin(70, 33, 1), seed=100 + bs)
    _check(step, waves=waves)


@pytest.mark.parametrize("waves", WAVES)
def test_prefill_unit_boundaries_and_group_sizes(waves) -> None:
    # 37 queries x 7 heads = 259 columns: two units, the second with 3 columns;
    # the group of 7 splits queries across column tiles and units.
    _announce(f"prefill unit boundaries waves={waves}")
    step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=[64, 0],
                     layouts=_lin(37, 73), seed=7)
    _check(step, waves=waves)


@pytest.mark.parametrize("waves", WAVES)
def test_prefill_tree_visibility(waves) -> None:
    _announce(f"prefill tree waves={waves}")
    rng = np.random.default_rng(11)
    parents = tuple([-1] + [int(rng.integers(0, i)) for i in range(1, 40)])
    step = make_step(hq=12, hkv=2, d=128, bs=16, dtype=torch.bfloat16, computed=[100, 33],
                     layouts=[parents, tuple(range(-1, 20))], seed=11)
    _check(step, waves=waves)


def test_prefill_lookahead_slots_are_not_read() -> None:
    _announce("prefill lookahead poison")
    step = make_step(hq=8, hkv=2, d=128, bs=4, dtype=torch.bfloat16, computed=[10, 3],
                     layouts=_lin(30, 20), reserved=[37, 26], num_blocks=40, seed=3)
    layer = step.cache.layer(step.layer_ids[0])
    slots = set(step.metadata.slot_mapping(block_size=4, device=DEV).tolist())
    flat_k = layer.keys.view(-1, 2, 128)
    flat_v = layer.values.view(-1, 2, 128)
    written = set()
    for table, c in zip(step.metadata.block_tables, step.metadata.num_computed_tokens):
        for pos in range(c):
            written.add(table[pos // 4] * 4 + pos % 4)
    poison = torch.tensor([s for s in range(flat_k.shape[0]) if s not in slots and s not in written], device=DEV)
    flat_k[poison] = float("nan")
    flat_v[poison] = float("nan")
    _check(step)


@pytest.mark.parametrize("waves", WAVES)
def test_c3_shape_mixed_batch(waves) -> None:
    # BASELINE C3 at reduced batch: 2 prefill chunks of 512 queries with prior
    # context, plus 6 decode tokens, Qwen2.5-7B attention shape.
    _announce(f"C3-shape mixed batch waves={waves}")
    rng = np.random.default_rng(3)
    computed = [int(c) for c in rng.integers(0, 3073, size=2)] + [int(c) for c in rng.integers(256, 4097, size=6)]
    step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=computed,
                     layouts=_lin(512, 512, *([1] * 6)), seed=3)
    _check(step, dense=True, waves=waves)


@pytest.mark.parametrize("waves", WAVES)
def test_per_xcd_orders_give_identical_outputs(waves) -> None:
    # The per-XCD order only decides which workgroup runs which unit (and
    # adds padding records): the grouped and plain orders give bit-identical
    # outputs, each also checked against the oracle.
    _announce(f"per-XCD orders waves={waves}")
    rng = np.random.default_rng(31)
    computed = [int(c) for c in rng.integers(0, 2000, size=5)]
    step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=computed,
                     layouts=_lin(*(int(q) for q in rng.integers(100, 420, size=5))), seed=31)
    outs, units = {}, {}
    for order in ("grouped", "plain"):
        backend = lv.HipPagedAttentionBackend(prefill_waves=waves, prefill_order=order)
        outs[order] = _check(step, backend=backend, waves=waves)
        ctx = backend.create(step.cache, step.metadata)
        units[order] = ctx.work_of(step.cache.layer_spec(step.layer_ids[0])).prefill_units.numpy()
    assert units["grouped"].tolist() != units["plain"].tolist()
    assert torch.equal(outs["grouped"], outs["plain"])


def test_prefill_kernel_agrees_with_the_decode_path() -> None:
    _announce("prefill vs decode path")
    step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=[200, 0],
                     layouts=_lin(64, 48), seed=8)
    a = _check(step)
    b = _check(step, backend=lv.HipPagedAttentionBackend(use_prefill_kernel=False), expect_prefill=False)
    assert (a.float() - b.float()).abs().max().item() <= 2e-2


def test_fp32_layers_use_the_decode_kernel() -> None:
    _announce("fp32 long queries")
    step = make_step(hq=4, hkv=2, d=64, bs=16, dtype=torch.float32, computed=[20], layouts=_lin(40), seed=5)
    _check(step, expect_prefill=False)


# ------------------------------------------------------ split-K prefill (key-range pieces + merge)
def _tree(rng, n):
    parents = [-1] + [int(rng.integers(0, i)) for i in range(1, n - 1)]
    return tuple([-1] + [0 if p == -1 else p + 1 for p in parents])  # 1 input token + (n-1)-node tree


def _split_work(step, waves=None):
    backend = lv.HipPagedAttentionBackend(prefill_waves=waves)
    ctx = backend.create(step.cache, step.metadata)
    return backend, ctx.work_of(step.cache.layer_spec(step.layer_ids[0]))


@pytest.mark.parametrize("waves", WAVES)
@pytest.mark.parametrize("dtype", ("bf16", "fp16"))
@pytest.mark.parametrize("head_size", range(32, 257, 16))
def test_split_k_tree_verification_head_sizes(dtype, head_size, waves) -> None:
    _announce(f"split-K prefill tree d={head_size} {dtype} waves={waves}")
    rng = np.random.default_rng(head_size)
    step = make_step(hq=12, hkv=2, d=head_size, bs=16, dtype=DTYPES[dtype], computed=[900, 1500, 370, 2100],
                     layouts=[_tree(rng, 9) for _ in range(4)], seed=head_size + 31)
    backend, work = _split_work(step, waves)
    assert work.num_prefill_partial_slots > 0 and work.num_prefill_jobs == 4
    assert work.prefill_waves == (waves if head_size <= 128 else 4)
    _check(step, backend=backend)


SPAN_CASES = {
    # name: (hq, hkv, d, bs, dtype, group prefix blocks, requests per group, decode rows between)
    "c5_bf16": (12, 2, 128, 16, "bf16", (128,), 12, False),
    "two_groups_bs12": (12, 2, 128, 12, "bf16", (60, 25), 6, True),
    "fp16_d64": (16, 2, 64, 16, "fp16", (40, 9), 5, True),
    "d256": (8, 2, 256, 16, "bf16", (33,), 6, False),
    "d80_group4": (16, 4, 80, 16, "fp16", (20,), 7, True),
}


@pytest.mark.parametrize("waves", WAVES)
@pytest.mark.parametrize("name", sorted(SPAN_CASES))
def test_shared_prefix_spans_match_the_oracle(name, waves) -> None:
    """Requests in groups sharing readonly prefixes (draft trees, causal
    chunks, decode rows between the groups): the spans' prefix attention plus
    each member's own keys, merged, equals the oracle, and equals the step
    planned without spans."""

    hq, hkv, d, bs, dtype, prefixes, per_group, decode_between = SPAN_CASES[name]
    _announce(f"shared-prefix spans {name} waves={waves}")
    rng = np.random.default_rng(len(name) * 31 + waves)
    layouts, computed, groups = [], [], []
    for g, blocks in enumerate(prefixes):
        for i in range(per_group):
            layouts.append(_tree(rng, 9) if i % 3 else _lin(int(rng.integers(3, 20)))[0])
            computed.append(blocks * bs + int(rng.integers(0, 300)))
            groups.append(g)
        if decode_between:
            layouts.append((-1,))
            computed.append(int(rng.integers(1, 900)))
            groups.append(-1)
    step = make_step(hq=hq, hkv=hkv, d=d, bs=bs, dtype=DTYPES[dtype], computed=computed, layouts=layouts,
                     prefix_groups=groups, group_prefix_blocks=prefixes, seed=len(name) + 900)
    backend = lv.HipPagedAttentionBackend(prefill_waves=waves)
    _, work = backend, backend.create(step.cache, step.metadata).work_of(step.cache.layer_spec(step.layer_ids[0]))
    assert (work.prefill_units.numpy()[:, 0] < 0).any(), "the step must use shared-prefix spans"
    out = _check(step, backend=lv.HipPagedAttentionBackend(prefill_waves=waves))
    plain = lv.HipPagedAttentionBackend(prefill_waves=waves, shared_prefix=False)
    ref = plain.create(step.cache, step.metadata).forward(step.layer_ids[0], step.query, step.key, step.value,
                                                          scale=step.scale)
    torch.cuda.synchronize()
    max_tol, _ = tolerances(step.query.dtype)
    assert (out.float() - ref.float()).abs().max().item() <= max_tol


def test_split_k_c5_shape_shared_prefix() -> None:
    # BASELINE C5 at reduced batch: 8 requests share a 2048-token prefix,
    # private suffixes, 9-token trees (1 input + 8 drafts) at group 6.
    _announce("split-K C5 shape")
    rng = np.random.default_rng(55)
    computed = [2048 + int(rng.integers(64, 513)) for _ in range(8)]
    step = make_step(hq=12, hkv=2, d=128, bs=16, dtype=torch.bfloat16, computed=computed,
                     layouts=[_tree(rng, 9) for _ in range(8)], shared_prefix_blocks=128, seed=55)
    backend, work = _split_work(step)
    assert work.num_prefill_partial_slots > 0
    _check(step, backend=backend)


@pytest.mark.parametrize("waves", WAVES)
@pytest.mark.parametrize("bs", (1, 3, 12, 16))
def test_split_k_causal_chunks_and_block_sizes(bs, waves) -> None:
    # Causal chunks with long prior context: 40 x 7 = 280 columns (three units,
    # the last partial), split over keys; plus decode rows in the same step.
    _announce(f"split-K causal chunks bs={bs}")
    step = make_step(hq=28, hkv=4, d=128, bs=bs, dtype=torch.bfloat16, computed=[3000, 700, 1200],
                     layouts=_lin(40, 3, 1), seed=80 + bs)
    backend, work = _split_work(step, waves)
    assert work.num_prefill_partial_slots > 0 and work.waves_per_head > 0
    _check(step, backend=backend, dense=True)


def test_split_k_matches_the_unsplit_kernel() -> None:
    # The same step through split pieces and through whole units agrees
    # within the bf16 tolerance (both are checked against the oracle too).
    _announce("split-K vs whole units")
    rng = np.random.default_rng(90)
    step = make_step(hq=12, hkv=2, d=128, bs=16, dtype=torch.bfloat16, computed=[1800, 2500],
                     layouts=[_tree(rng, 9), _tree(rng, 9)], seed=90)
    backend, work = _split_work(step)
    assert work.num_prefill_partial_slots > 0
    a = _check(step, backend=backend)
    whole = lv.HipPagedAttentionBackend(split_prefill=False)
    ctx = whole.create(step.cache, step.metadata)
    w2 = ctx.work_of(step.cache.layer_spec(step.layer_ids[0]))
    real = int((w2.prefill_units.numpy()[:, 2] > 0).sum())  # (the rest pads the per-XCD order)
    assert w2.num_prefill_partial_slots == 0 and real == 2
    b = _check(step, backend=whole)
    assert (a.float() - b.float()).abs().max().item() <= 2e-2
