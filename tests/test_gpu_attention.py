"""GPU parity of HIP paged attention against the CPU oracle.

Tolerances (written per dtype in paged_cases.tolerances): bf16 max-abs 2e-2 /
mean-abs 2e-3, fp32 max-abs 1e-5, fp16 3e-3 / 3e-4.  Every case also checks
that this step's K/V landed bit-exactly at its slots (write before attend).
The reference's own Triton GPU tests (tests/test_triton_paged_attention.py:
101-278) are mirrored case for case, then the BASELINE shapes.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import light_vllm_amd as lv
from paged_cases import DTYPES, make_step, oracle_attention, report_margin, tolerances

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

DEV = torch.device("cuda:0")


def _announce(name: str) -> None:
    print(f"[gpu] {name}", file=sys.stderr, flush=True)


def _run_and_check(step, *, backend=None, layer_index: int = 0, margin: str | None = None):
    backend = backend or lv.HipPagedAttentionBackend()
    ctx = backend.create(step.cache, step.metadata)
    lid = step.layer_ids[layer_index]
    out = ctx.forward(lid, step.query, step.key, step.value, scale=step.scale)
    torch.cuda.synchronize()
    assert out.shape == step.query.shape and out.dtype == step.query.dtype
    # Write-then-attend: this step's K/V sit at their slots, bit for bit.
    slots = step.metadata.slot_mapping(block_size=step.cache.config.block_size, device=DEV)
    layer = step.cache.layer(lid)
    nslots = step.cache.config.num_blocks * step.cache.config.block_size
    hkv, d = step.key.shape[1:]
    assert torch.equal(layer.keys.view(nslots, hkv, d).index_select(0, slots), step.key)
    assert torch.equal(layer.values.view(nslots, hkv, d).index_select(0, slots), step.value)
    expect = oracle_attention(step, lid)
    got = out.float().cpu().numpy()
    err = np.abs(got - expect)
    max_tol, mean_tol = tolerances(step.query.dtype)
    if margin is not None:
        report_margin(margin, err, step.query.dtype)
    assert np.isfinite(got).all()
    assert err.max() <= max_tol, f"max-abs {err.max():.3e} > {max_tol}"
    assert err.mean() <= mean_tol, f"mean-abs {err.mean():.3e} > {mean_tol}"
    return out, ctx


def _lin(*lengths):
    return [tuple(range(-1, n - 1)) for n in lengths]


# ------------------------------------------------------ mirrors of the reference's Triton tests
@pytest.mark.parametrize("head_size", (32, 80, 128, 256))
@pytest.mark.parametrize("dtype", ("fp16", "bf16"))
def test_packed_gqa_prefill(head_size, dtype) -> None:
    _announce(f"packed gqa prefill d={head_size} {dtype}")
    step = make_step(hq=4, hkv=2, d=head_size, bs=4, dtype=DTYPES[dtype], computed=[0, 0],
                     layouts=_lin(6, 3), num_blocks=16, seed=20260817)
    _run_and_check(step)


def test_qwen_gqa_group() -> None:
    _announce("qwen gqa group")
    step = make_step(hq=28, hkv=4, d=128, bs=4, dtype=torch.bfloat16, computed=[0, 0],
                     layouts=_lin(6, 3), num_blocks=16, seed=20260822)
    _run_and_check(step)


def test_qwen_gqa_across_history_chunks() -> None:
    _announce("qwen gqa history 130")
    step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=[130],
                     layouts=_lin(1), num_blocks=16, seed=20260822)
    _run_and_check(step)


def test_packed_tree_visibility() -> None:
    _announce("tree visibility")
    step = make_step(hq=4, hkv=2, d=64, bs=2, dtype=torch.float16, computed=[0, 0],
                     layouts=[(-1, 0, 0, 2), (-1, 0, 0)], num_blocks=16, seed=20260819)
    _run_and_check(step)


def test_decode_after_prefill_reads_the_prefill_kv() -> None:
    _announce("decode after prefill")
    backend = lv.HipPagedAttentionBackend()
    step = make_step(hq=4, hkv=2, d=64, bs=2, dtype=torch.float16, computed=[0, 0],
                     layouts=_lin(5, 3), num_blocks=16, seed=20260817)
    _run_and_check(step, backend=backend)
    tables = step.metadata.block_tables
    decode_md = lv.PagedAttentionMetadata(block_tables=tables, num_computed_tokens=(5, 3),
                                          query_layouts=tuple(lv.linear_query_layout(1) for _ in range(2)))
    gen = torch.Generator(device="cpu").manual_seed(1)
    step.metadata = decode_md
    step.query = torch.randn((2, 4, 64), generator=gen).half().to(DEV)
    step.key = torch.randn((2, 2, 64), generator=gen).half().to(DEV)
    step.value = torch.randn((2, 2, 64), generator=gen).half().to(DEV)
    _run_and_check(step, backend=backend)


def test_shared_readonly_prefix() -> None:
    _announce("shared readonly prefix")
    step = make_step(hq=4, hkv=2, d=64, bs=2, dtype=torch.float16, computed=[2, 2],
                     layouts=_lin(1, 1), num_blocks=16, shared_prefix_blocks=1, seed=20260817)
    assert step.metadata.block_tables[0][0] == step.metadata.block_tables[1][0]
    _run_and_check(step)


def test_unused_lookahead_slots_are_not_read_or_written() -> None:
    _announce("unused lookahead")
    step = make_step(hq=4, hkv=2, d=64, bs=2, dtype=torch.float16, computed=[0, 0],
                     layouts=_lin(3, 1), reserved=[5, 4], num_blocks=16, seed=20260817)
    layer = step.cache.layer(step.layer_ids[0])
    # Poison every slot outside this step's writes: a read of an unused slot would show.
    slots = set(step.metadata.slot_mapping(block_size=2, device=DEV).tolist())
    flat_k = layer.keys.view(-1, 2, 64)
    flat_v = layer.values.view(-1, 2, 64)
    poison = torch.tensor([s for s in range(flat_k.shape[0]) if s not in slots], device=DEV)
    flat_k[poison] = float("nan")
    flat_v[poison] = float("nan")
    before = flat_k[poison].clone()
    _run_and_check(step)
    assert torch.equal(flat_k[poison].isnan(), before.isnan())


# ------------------------------------------------------ BASELINE shapes
def test_c1_qwen05b_fp32_decode() -> None:
    _announce("C1 fp32 decode")
    step = make_step(hq=14, hkv=2, d=64, bs=16, dtype=torch.float32, computed=[37, 128, 200, 511],
                     layouts=_lin(1, 1, 1, 1), num_blocks=256, seed=1)
    _run_and_check(step, margin="C1 (fp32, stream-K)")


def test_c2_qwen7b_bf16_decode_bs64() -> None:
    _announce("C2 bf16 decode bs64")
    rng = np.random.default_rng(2)
    ctx = [int(c) for c in rng.integers(512, 4097, size=64)]
    step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=ctx,
                     layouts=_lin(*([1] * 64)), num_blocks=32768, seed=2)
    _, ctx_obj = _run_and_check(step, margin="C2 (bf16, stream-K, bf16 partials)")
    work = ctx_obj.work_of(step.cache.layer_spec(step.layer_ids[0]))
    assert work.num_jobs > 0 and work.group_waves == 1, "C2 must exercise the split-K merge"


def test_small_batch_reference_point_bf16() -> None:
    # The reference's published operating point: B=16, context 256, Qwen2.5-7B.
    _announce("small batch bf16 decode (B=16, ctx 256)")
    step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=[256] * 16,
                     layouts=_lin(*([1] * 16)), num_blocks=1024, seed=16)
    _, ctx_obj = _run_and_check(step, margin="small (bf16, workgroup split)")
    assert ctx_obj.work_of(step.cache.layer_spec(step.layer_ids[0])).group_waves > 1


@pytest.mark.parametrize("dtype", ("fp32", "fp16", "bf16"))
@pytest.mark.parametrize("head_size", range(32, 257, 16))
def test_head_sizes_and_dtypes_decode_with_split_k(dtype, head_size) -> None:
    _announce(f"decode d={head_size} {dtype}")
    step = make_step(hq=8, hkv=2, d=head_size, bs=16, dtype=DTYPES[dtype], computed=[700, 3, 1500, 64],
                     layouts=_lin(1, 1, 1, 2), seed=head_size)
    _run_and_check(step)


@pytest.mark.parametrize("bs", (1, 2, 3, 4, 32))
def test_block_sizes(bs) -> None:
    _announce(f"block size {bs}")
    step = make_step(hq=12, hkv=2, d=128, bs=bs, dtype=torch.bfloat16, computed=[45, 300, 0],
                     layouts=_lin(1, 3, 7), seed=bs)
    _run_and_check(step)


def test_tree_verification_with_shared_prefix_c5_shape() -> None:
    _announce("C5-shape tree verify")
    rng = np.random.default_rng(5)
    layouts, computed = [], []
    for _ in range(8):
        parents = [-1] + [int(rng.integers(0, i)) for i in range(1, 8)]
        layouts.append(tuple([-1] + [0 if p == -1 else p + 1 for p in parents]))  # 1 input + 8-node tree
        computed.append(2048 + int(rng.integers(64, 513)))
    step = make_step(hq=12, hkv=2, d=128, bs=16, dtype=torch.bfloat16, computed=computed, layouts=layouts,
                     shared_prefix_blocks=128, seed=5)
    _run_and_check(step)


def test_long_queries_through_every_column_tile() -> None:
    _announce("long queries")
    step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=[0, 300, 1000],
                     layouts=_lin(40, 17, 70), seed=9)
    _run_and_check(step)


def test_every_layer_runs_once_and_layer_ids_are_reported() -> None:
    step = make_step(hq=4, hkv=2, d=64, bs=16, dtype=torch.bfloat16, computed=[10], layouts=_lin(1),
                     num_layers=2, seed=3)
    ctx = lv.HipPagedAttentionBackend().create(step.cache, step.metadata)
    ctx.forward("layer0", step.query, step.key, step.value, scale=step.scale)
    with pytest.raises(lv.KVCacheError, match="ran more than once"):
        ctx.forward("layer0", step.query, step.key, step.value, scale=step.scale)
    ctx.forward("layer1", step.query, step.key, step.value, scale=step.scale)
    assert ctx.layer_ids == frozenset({"layer0", "layer1"})


def test_shape_and_dtype_validation() -> None:
    step = make_step(hq=4, hkv=2, d=64, bs=16, dtype=torch.bfloat16, computed=[10], layouts=_lin(2), seed=3)
    ctx = lv.HipPagedAttentionBackend().create(step.cache, step.metadata)
    with pytest.raises(lv.KVCacheError, match="token count does not match"):
        ctx.forward("layer0", step.query[:1], step.key[:1], step.value[:1], scale=step.scale)
    ctx = lv.HipPagedAttentionBackend().create(step.cache, step.metadata)
    with pytest.raises(lv.KVCacheError, match="dtype and device must match"):
        ctx.forward("layer0", step.query.float(), step.key, step.value, scale=step.scale)


@pytest.mark.parametrize("partition", (32, 512, 2048))
@pytest.mark.parametrize("bs", (1, 16))
def test_partition_caps_within_the_lds_table_slice(partition, bs) -> None:
    # A wave's table slice lives in LDS (256 entries).  At bs=1 a 512- or
    # 2048-token partition would need more entries, so the planner cuts the
    # shares at the slice instead (254 blocks after alignment): every share,
    # whatever the partition asks for, must fit, and the result must hold.
    _announce(f"partition {partition} bs {bs}")
    step = make_step(hq=28, hkv=4, d=128, bs=bs, dtype=torch.bfloat16, computed=[1200, 37, 2600],
                     layouts=_lin(1, 2, 1), seed=partition + bs)
    backend = lv.HipPagedAttentionBackend(partition_tokens=partition)
    work = backend.create(step.cache, step.metadata).work_of(step.cache.layer_spec(step.layer_ids[0]))
    unit = lv.native.decode_tile_tokens(lv.native.DTYPE_BF16, 128, work.col_tiles)
    assert work.units_per_wave * unit <= min(partition, 254 * bs)
    _run_and_check(step, backend=backend)



def test_two_split_k_layers_share_the_workspace() -> None:
    _announce("two split-K layers")
    backend = lv.HipPagedAttentionBackend()
    step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=[3000, 1700, 40],
                     layouts=_lin(1, 1, 1), num_layers=2, seed=21)
    ctx = backend.create(step.cache, step.metadata)
    assert ctx.plan.work(7, 4, lv.native.resident_decode_waves(2, 128)).num_jobs > 0
    max_tol, mean_tol = tolerances(step.query.dtype)
    for layer_index in range(2):
        lid = step.layer_ids[layer_index]
        out = ctx.forward(lid, step.query, step.key, step.value, scale=step.scale)
        torch.cuda.synchronize()
        err = np.abs(out.float().cpu().numpy() - oracle_attention(step, lid))
        assert err.max() <= max_tol and err.mean() <= mean_tol


@pytest.mark.parametrize("prefill", (False, True))
def test_split_k_partials_hold_values_near_the_fp16_limit(prefill) -> None:
    # Split-K partials are stored in the pool's type, normalised by their own
    # softmax sums: a convex combination of V rows, so fp16 partials cannot
    # overflow while |V| stays below the fp16 maximum.  V of magnitude up to
    # about 4.5e4 (65504 is the largest fp16), split decode rows and split
    # tree verification over a shared prefix; errors relative to the scale.
    # (Only the pool's written history is scaled into range; slots nothing
    # wrote may hold anything and are never read.)
    _announce(f"fp16 partials near the limit prefill={prefill}")
    scale_v = 8.0e3
    rng = np.random.default_rng(77)
    if prefill:
        layouts = []
        for _ in range(4):  # the input token, then an 8-node draft tree under it
            parents = [-1] + [int(rng.integers(0, i)) for i in range(1, 8)]
            layouts.append(tuple([-1] + [0 if q == -1 else q + 1 for q in parents]))
        step = make_step(hq=12, hkv=2, d=128, bs=16, dtype=torch.float16,
                         computed=[2048 + int(c) for c in rng.integers(64, 513, size=4)],
                         layouts=layouts, shared_prefix_blocks=128, seed=77)
    else:
        step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.float16, computed=[3000, 1700, 2500],
                         layouts=_lin(1, 1, 1), seed=78)
    lid = step.layer_ids[0]
    step.cache.layer(lid).values.mul_(scale_v)
    step.value.mul_(scale_v)
    assert torch.isfinite(step.value).all()
    ctx = lv.HipPagedAttentionBackend().create(step.cache, step.metadata)
    out = ctx.forward(lid, step.query, step.key, step.value, scale=step.scale)
    torch.cuda.synchronize()
    expect = oracle_attention(step, lid)  # (after the forward: the oracle reads the appended rows)
    assert np.isfinite(expect).all()
    work = ctx.work_of(step.cache.layer_spec(lid))
    assert (work.num_prefill_jobs if prefill else work.num_jobs) > 0, "the step must write split-K partials"
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    err = np.abs(got - expect) / scale_v
    max_tol, mean_tol = tolerances(torch.float16)
    assert err.max() <= max_tol and err.mean() <= mean_tol, (err.max(), err.mean())


# ------------------------------------------------------ four column tiles per decode wave
@pytest.mark.parametrize("dtype", ("fp32", "fp16", "bf16"))
@pytest.mark.parametrize("head_size", (32, 48, 64, 80, 96, 112, 128))
def test_four_column_tiles_across_dtypes_and_head_sizes(dtype, head_size) -> None:
    # Eight queries x group 4 = 32 columns: two column tiles of a four-tile group.
    _announce(f"col_tiles=4 d={head_size} {dtype}")
    step = make_step(hq=8, hkv=2, d=head_size, bs=16, dtype=DTYPES[dtype], computed=[700, 3, 1500, 64],
                     layouts=_lin(8, 1, 9, 2), seed=head_size + 5)
    _run_and_check(step, backend=lv.HipPagedAttentionBackend(use_prefill_kernel=False, decode_col_tiles=4))


@pytest.mark.parametrize("col_tiles", (1, 4))
@pytest.mark.parametrize("partition", (None, 32))
def test_tree_verification_by_column_tiles(col_tiles, partition) -> None:
    # 9-token trees at group 7 = 63 columns: four column tiles, split into
    # many partials when partitions are short.
    _announce(f"tree verify col_tiles={col_tiles} partition={partition}")
    rng = np.random.default_rng(51)
    layouts, computed = [], []
    for _ in range(6):
        parents = [-1] + [int(rng.integers(0, i)) for i in range(1, 8)]
        layouts.append(tuple([-1] + [0 if p == -1 else p + 1 for p in parents]))
        computed.append(256 + int(rng.integers(0, 900)))
    step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=computed, layouts=layouts,
                     shared_prefix_blocks=16, seed=52)
    backend = lv.HipPagedAttentionBackend(use_prefill_kernel=False, decode_col_tiles=col_tiles,
                                          partition_tokens=partition)
    _, ctx = _run_and_check(step, backend=backend)
    work = ctx.plan.work(7, 4, lv.native.resident_decode_waves(2, 128, col_tiles), 0,
                         lv.native.decode_tile_tokens(2, 128, col_tiles), col_tiles)
    assert work.col_tiles == col_tiles


@pytest.mark.parametrize("bs", (1, 3, 16))
def test_four_column_tiles_long_queries_without_prefill_kernel(bs) -> None:
    # 40 queries x group 7 = 280 columns = 18 column tiles: four full groups
    # and a partial one, all through the decode kernel.
    _announce(f"col_tiles=4 long queries bs={bs}")
    step = make_step(hq=28, hkv=4, d=128, bs=bs, dtype=torch.bfloat16, computed=[0, 300, 1000],
                     layouts=_lin(40, 17, 5), seed=60 + bs)
    backend = lv.HipPagedAttentionBackend(use_prefill_kernel=False, decode_col_tiles=4, partition_tokens=256)
    _run_and_check(step, backend=backend)


def test_auto_column_tiles_pick_four_for_trees_and_one_for_decode() -> None:
    # Without the prefill kernel (as for fp32 layers) multi-tile rows take
    # the four-column-tile decode kernel.
    _announce("auto column tiles")
    step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=[500, 900],
                     layouts=_lin(8, 8), seed=71)
    _, ctx = _run_and_check(step, backend=lv.HipPagedAttentionBackend(use_prefill_kernel=False))
    assert ctx.plan.choose_col_tiles(7, 0, 4) == 4
    step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=[500, 900],
                     layouts=_lin(1, 1), seed=72)
    _, ctx = _run_and_check(step)
    assert ctx.plan.choose_col_tiles(7, 0, 4) == 1


# ------------------------------------------------------ in-launch merge, fast path, plan reuse
def _forward_error(step, lid, out) -> tuple[float, float]:
    err = np.abs(out.float().cpu().numpy() - oracle_attention(step, lid))
    return float(err.max()), float(err.mean())


def test_fused_qkv_views_take_either_path() -> None:
    # q, k and v as views of one fused projection row [T, (Hq + 2 Hkv) D]:
    # aligned views go through the one-call path, a view whose rows start
    # two bytes in goes through the general path (copied to aligned rows).
    _announce("fused qkv views")
    step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=[900, 40, 2100],
                     layouts=_lin(1, 1, 1), num_layers=2, seed=311)
    t, hq, d = step.query.shape
    hkv = step.key.shape[1]
    width = (hq + 2 * hkv) * d
    ctx = lv.HipPagedAttentionBackend().create(step.cache, step.metadata)
    for lid, shift in zip(step.layer_ids, (0, 1)):
        fused = torch.zeros((t, width + 8), dtype=step.query.dtype, device=DEV)
        body = fused[:, shift : shift + width]
        body[:, : hq * d] = step.query.reshape(t, -1)
        body[:, hq * d : (hq + hkv) * d] = step.key.reshape(t, -1)
        body[:, (hq + hkv) * d :] = step.value.reshape(t, -1)
        q = body[:, : hq * d].view(t, hq, d)
        k = body[:, hq * d : (hq + hkv) * d].view(t, hkv, d)
        v = body[:, (hq + hkv) * d :].view(t, hkv, d)
        assert not q.is_contiguous()
        out = ctx.forward(lid, q, k, v, scale=step.scale)
        torch.cuda.synchronize()
        mx, mean = _forward_error(step, lid, out)
        max_tol, mean_tol = tolerances(step.query.dtype)
        assert mx <= max_tol and mean <= mean_tol, (lid, shift, mx, mean)


def test_one_metadata_on_caches_of_two_dtypes() -> None:
    # A plan is reused only by a cache of the same geometry, dtype and layer
    # shapes: the same metadata object sent to a bf16 cache and then to an
    # fp16 cache of equal geometry must run each cache's own kernels; back on
    # the bf16 cache it is planned again, and a second create() on that same
    # cache takes the plan by identity.
    _announce("one metadata, two dtypes")
    step = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=[1500, 33, 700],
                     layouts=_lin(1, 9, 1), seed=321)
    lid = step.layer_ids[0]
    config = step.cache.config
    spec = lv.ModelKVCacheSpec((lv.AttentionLayerSpec(lid, 28, 4, 128),))
    cache16 = lv.PagedKVCache(spec, lv.PagedKVCacheConfig(num_blocks=config.num_blocks, block_size=config.block_size,
                                                          dtype=torch.float16, device=DEV))
    src = step.cache.layer(lid)
    cache16.layer(lid).keys.copy_(src.keys.to(torch.float16))
    cache16.layer(lid).values.copy_(src.values.to(torch.float16))
    step16 = type(step)(cache16, step.metadata, step.query.to(torch.float16), step.key.to(torch.float16),
                        step.value.to(torch.float16), step.layer_ids, step.scale)
    backend = lv.HipPagedAttentionBackend()
    for s in (step, step16, step, step):
        ctx = backend.create(s.cache, s.metadata)
        out = ctx.forward(lid, s.query, s.key, s.value, scale=s.scale)
        torch.cuda.synchronize()
        assert out.dtype == s.query.dtype
        mx, mean = _forward_error(s, lid, out)
        max_tol, mean_tol = tolerances(s.query.dtype)
        assert mx <= max_tol and mean <= mean_tol, (s.query.dtype, mx, mean)


def test_layers_of_two_shapes_alternating_in_one_cache() -> None:
    # forward binds the fast path once per layer shape and step (plan and
    # output slab) and passes each layer's pools and output rows on their
    # own: layers of two shapes, interleaved, each match the oracle; the
    # outputs are distinct rows, later layers leave earlier outputs alone,
    # and a second step on the same metadata (the plan reused, new slabs)
    # leaves the first step's outputs alone too.
    _announce("two layer shapes, alternating")
    base = make_step(hq=28, hkv=4, d=128, bs=16, dtype=torch.bfloat16, computed=[700, 40, 1500, 0],
                     layouts=_lin(1, 9, 1, 33), seed=401)
    config = base.cache.config
    shapes = {"a0": (28, 4, 128), "b0": (12, 2, 64), "a1": (28, 4, 128), "b1": (12, 2, 64)}
    spec = lv.ModelKVCacheSpec(tuple(lv.AttentionLayerSpec(lid, *shape) for lid, shape in shapes.items()))
    cache = lv.PagedKVCache(spec, lv.PagedKVCacheConfig(num_blocks=config.num_blocks, block_size=config.block_size,
                                                        dtype=config.dtype, device=DEV))
    gen = torch.Generator(device=DEV).manual_seed(402)
    for lid in shapes:
        layer = cache.layer(lid)
        layer.keys.copy_(torch.randn(layer.keys.shape, generator=gen, device=DEV).to(config.dtype))
        layer.values.copy_(torch.randn(layer.values.shape, generator=gen, device=DEV).to(config.dtype))
    t = base.query.shape[0]

    def inputs(lid):
        hq, hkv, d = shapes[lid]
        q = torch.randn((t, hq, d), generator=gen, device=DEV).to(config.dtype)
        k = torch.randn((t, hkv, d), generator=gen, device=DEV).to(config.dtype)
        v = torch.randn((t, hkv, d), generator=gen, device=DEV).to(config.dtype)
        return q, k, v, 1.0 / float(np.sqrt(d))

    step_inputs = {lid: inputs(lid) for lid in shapes}
    backend = lv.HipPagedAttentionBackend()
    ctx = backend.create(cache, base.metadata)
    outs = {lid: ctx.forward(lid, *step_inputs[lid][:3], scale=step_inputs[lid][3]) for lid in shapes}
    torch.cuda.synchronize()
    assert len({o.data_ptr() for o in outs.values()}) == len(outs)
    max_tol, mean_tol = tolerances(config.dtype)
    first = {}
    for lid, out in outs.items():
        q, k, v, scale = step_inputs[lid]
        assert out.shape == q.shape and out.dtype == q.dtype
        check = type(base)(cache, base.metadata, q, k, v, (lid,), scale)
        mx, mean = _forward_error(check, lid, out)
        assert mx <= max_tol and mean <= mean_tol, (lid, mx, mean)
        first[lid] = out.clone()
    # The same step again (same K/V, new queries): new outputs, old ones kept.
    ctx2 = backend.create(cache, base.metadata)
    again = {}
    for lid in shapes:
        q, k, v, scale = step_inputs[lid]
        again[lid] = ctx2.forward(lid, -q, k, v, scale=scale)
    torch.cuda.synchronize()
    for lid in shapes:
        assert torch.equal(outs[lid], first[lid]), lid
        assert again[lid].data_ptr() != outs[lid].data_ptr()
        q, k, v, scale = step_inputs[lid]
        check = type(base)(cache, base.metadata, -q, k, v, (lid,), scale)
        mx, mean = _forward_error(check, lid, again[lid])
        assert mx <= max_tol and mean <= mean_tol, (lid, mx, mean)


# ------------------------------------------------------ workgroup split (latency-bound decode)
@pytest.mark.parametrize("dtype", ("fp32", "fp16", "bf16"))
@pytest.mark.parametrize("head_size", range(32, 257, 16))
def test_workgroup_split_decode_matches_the_oracle(dtype, head_size) -> None:
    # Short decode rows (one segment per workgroup of eight waves, four for
    # the widest rows, results combined in LDS): a 1-token context, segments
    # of fewer tiles than waves (idle waves) and of more (up to the 1.5 tiles
    # per wave the planner splits at), append fused.
    _announce(f"workgroup split d={head_size} {dtype}")
    hq, hkv = (28, 4) if head_size <= 128 else (16, 2)
    code = lv.paged_cache.dtype_code(DTYPES[dtype])
    unit, gw = lv.native.decode_tile_tokens(code, head_size), lv.native.decode_split_waves(code, head_size)
    computed = [0, unit - 1, unit + 8, (3 * gw // 2) * unit - 1, gw * unit - 1, 2 * unit + 3, 3 * unit, 5]
    step = make_step(hq=hq, hkv=hkv, d=head_size, bs=16, dtype=DTYPES[dtype], computed=computed,
                     layouts=_lin(*([1] * 8)), seed=400 + head_size)
    _, ctx = _run_and_check(step)
    work = ctx.work_of(step.cache.layer_spec(step.layer_ids[0]))
    assert work.group_waves == gw > 1 and work.num_jobs == 0 and work.units_per_wave == 2


@pytest.mark.parametrize("dtype", ("fp32", "bf16"))
def test_workgroup_split_of_multi_tile_rows_without_prefill_kernel(dtype) -> None:
    # Query runs wider than one column tile through the decode kernel (as
    # for fp32 layers): each (request, column tile) segment takes its own
    # workgroup, and the LDS merge writes that tile's columns.
    _announce(f"workgroup split, column tiles 1-5 {dtype}")
    step = make_step(hq=4, hkv=2, d=64, bs=16, dtype=DTYPES[dtype], computed=[20, 90, 3],
                     layouts=_lin(40, 9, 17), seed=420)
    backend = lv.HipPagedAttentionBackend(use_prefill_kernel=False, decode_col_tiles=1)
    _, ctx = _run_and_check(step, backend=backend)
    assert ctx.work_of(step.cache.layer_spec(step.layer_ids[0])).group_waves == 8


@pytest.mark.parametrize("bs", (1, 3, 16))
@pytest.mark.parametrize("hq,hkv", ((4, 4), (32, 4), (12, 2)))
def test_workgroup_split_block_sizes_and_groups(bs, hq, hkv) -> None:
    # Block sizes through the division path and the first-tile block ids,
    # group sizes 1, 8 and 6, against the oracle and the stream-K plan.
    _announce(f"workgroup split bs={bs} {hq}/{hkv}")
    step = make_step(hq=hq, hkv=hkv, d=128, bs=bs, dtype=torch.bfloat16, computed=[250, 17, 260, 3, 129],
                     layouts=_lin(1, 1, 1, 1, 1), num_layers=2, seed=410 + bs + hq)
    out, ctx = _run_and_check(step)
    assert ctx.work_of(step.cache.layer_spec(step.layer_ids[0])).group_waves == 8
    ref = lv.HipPagedAttentionBackend(decode_workgroups=False).create(step.cache, step.metadata)
    lid = step.layer_ids[1]
    # (layer1's pool holds this step's K/V only after the forward below)
    out1 = ctx.forward(lid, step.query, step.key, step.value, scale=step.scale)
    out2 = ref.forward(lid, step.query, step.key, step.value, scale=step.scale)
    torch.cuda.synchronize()
    assert ref.work_of(step.cache.layer_spec(lid)).group_waves == 1
    max_tol, _ = tolerances(step.query.dtype)
    assert (out1.float() - out2.float()).abs().max().item() <= max_tol


@pytest.mark.parametrize("head_size", (16, 40, 72, 264))
def test_unbuilt_head_sizes_are_refused_when_the_step_starts(head_size) -> None:
    # The kernels are built for head sizes that are multiples of 16 from 32
    # to 256; a cache with another layer shape fails at create() with the
    # reference's error class, before any layer's forward.
    spec = lv.ModelKVCacheSpec((lv.AttentionLayerSpec("a", 8, 2, 128), lv.AttentionLayerSpec("b", 8, 2, head_size)))
    cache = lv.PagedKVCache(spec, lv.PagedKVCacheConfig(num_blocks=8, block_size=16, dtype=torch.bfloat16, device=DEV))
    md = lv.PagedAttentionMetadata(block_tables=((0,),), num_computed_tokens=(3,),
                                   query_layouts=(lv.linear_query_layout(1),))
    with pytest.raises(lv.KVCacheError, match=f"not {head_size}"):
        lv.HipPagedAttentionBackend().create(cache, md)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ("bf16", "fp16"))
@pytest.mark.parametrize("bs", (1, 3, 12, 16, 32))
@pytest.mark.parametrize("partition", (None, 32))
def test_line_order_decode_tiles_at_every_row_offset(dtype, bs, partition) -> None:
    """The stream-K decode kernel's line-order tiles (16-bit pools, head size
    128): contexts that end at every row of a 32-token tile (a piece's last
    rows repeat its last key, masked), a fresh token landing on each row of
    its tile (the fused append writes it from the line-order registers), and
    one-tile shares (partition 32) so that pieces start and end inside
    segments.  Outputs against the oracle, pool slots bit for bit."""

    _announce(f"line-order decode {dtype} bs {bs} partition {partition}")
    computed = [0, 1, 2, 3, 4, 5, 15, 16, 17, 30, 31, 32, 33, 63, 64, 65, 100, 255, 300]
    step = make_step(hq=28, hkv=4, d=128, bs=bs, dtype=DTYPES[dtype], computed=computed,
                     layouts=_lin(*([1] * len(computed))), seed=4100 + bs)
    backend = lv.HipPagedAttentionBackend(partition_tokens=partition, decode_workgroups=False)
    _, ctx = _run_and_check(step, backend=backend)
    work = ctx.work_of(step.cache.layer_spec(step.layer_ids[0]))
    assert work.group_waves == 1 and work.col_tiles == 1  # the stream-K kernel, one column tile
    if partition:
        assert work.units_per_wave == 1
