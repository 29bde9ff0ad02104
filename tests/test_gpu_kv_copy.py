"""GPU parity of the KV movement kernels: append, compact, block copy.

All three must be bit-exact against the CPU oracle: full pools are compared
byte for byte (as integer views), so every untouched byte must be unchanged.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import light_vllm_amd as lv
from oracle import paged_kv_oracle as O

pytestmark = pytest.mark.gpu
if not torch.cuda.is_available():
    pytest.skip("needs an MI355X GPU", allow_module_level=True)

DEV = torch.device("cuda:0")
GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
INT_VIEW = {torch.float32: torch.int32, torch.float16: torch.int16, torch.bfloat16: torch.int16}


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.view(INT_VIEW[t.dtype]).cpu().numpy()


def _announce(name: str) -> None:
    print(f"[gpu] {name}", file=sys.stderr, flush=True)


def _cache(*, hkv, d, bs, nb, dtype, layers=1, hq=None):
    spec = lv.ModelKVCacheSpec(tuple(lv.AttentionLayerSpec(f"l{i}", hq or hkv, hkv, d) for i in range(layers)))
    cache = lv.PagedKVCache(spec, lv.PagedKVCacheConfig(num_blocks=nb, block_size=bs, dtype=dtype, device=DEV))
    gen = torch.Generator(device=DEV).manual_seed(nb * 7 + d)
    for i in range(layers):
        layer = cache.layer(f"l{i}")
        for pool in (layer.keys, layer.values):
            pool.copy_(torch.randn(pool.shape, generator=gen, device=DEV).to(dtype))
    return cache


@pytest.mark.parametrize(
    "name,hkv,d,bs,nb,dtype,tokens",
    [
        ("c1_fp32", 2, 64, 16, 256, torch.float32, 4),
        ("c2_bf16", 4, 128, 16, 32768, torch.bfloat16, 64),
        ("c3_bf16_4152", 4, 128, 16, 4096, torch.bfloat16, 4152),
        ("fp16_d80_bs3", 2, 80, 3, 64, torch.float16, 29),
    ],
)
def test_append_is_bit_exact(name, hkv, d, bs, nb, dtype, tokens) -> None:
    _announce(f"append {name}")
    cache = _cache(hkv=hkv, d=d, bs=bs, nb=nb, dtype=dtype)
    layer = cache.layer("l0")
    rng = np.random.default_rng(tokens)
    slots = rng.choice(nb * bs, size=tokens, replace=False)
    key = torch.randn((tokens, hkv, d)).to(dtype).to(DEV)
    value = torch.randn((tokens, hkv, d)).to(dtype).to(DEV)
    kb, vb = _bits(layer.keys), _bits(layer.values)
    O.append(kb, vb, _bits(key), _bits(value), slots)
    cache.write("l0", key, value, torch.tensor(slots, device=DEV))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(layer.keys), kb)
    np.testing.assert_array_equal(_bits(layer.values), vb)


def test_append_reads_strided_views_and_skips_inactive_tokens() -> None:
    _announce("append strided")
    hq, hkv, d = 28, 4, 128
    cache = _cache(hkv=hkv, d=d, bs=16, nb=64, dtype=torch.bfloat16, hq=hq)
    layer = cache.layer("l0")
    qkv = torch.randn((10, hq + 2 * hkv, d)).to(torch.bfloat16).to(DEV)  # fused QKV output
    key, value = qkv[:, hq : hq + hkv], qkv[:, hq + hkv :]
    assert not key.is_contiguous()
    slots = np.array([5, -1, 17, 900, -1, 0, 31, 640, 1023, 2])
    kb, vb = _bits(layer.keys), _bits(layer.values)
    O.append(kb, vb, _bits(key.contiguous()), _bits(value.contiguous()), slots)
    cache.write("l0", key, value, torch.tensor(slots, device=DEV))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(layer.keys), kb)
    np.testing.assert_array_equal(_bits(layer.values), vb)


def test_append_validation_matches_reference_errors() -> None:
    cache = _cache(hkv=2, d=64, bs=16, nb=8, dtype=torch.float32)
    k = torch.randn((2, 2, 64), device=DEV)
    with pytest.raises(lv.KVCacheError, match="out-of-range physical slot"):
        cache.write("l0", k, k, torch.tensor([0, 128], device=DEV))
    with pytest.raises(lv.KVCacheError, match="same physical slot twice"):
        cache.write("l0", k, k, torch.tensor([3, 3], device=DEV))
    with pytest.raises(lv.KVCacheError, match="dtype and device must match"):
        cache.write("l0", k.half(), k.half(), torch.tensor([0, 1], device=DEV))


def test_compact_known_answer_on_gpu() -> None:
    _announce("compact known answer")
    c = GOLDEN["compact"]
    spec = lv.ModelKVCacheSpec((lv.AttentionLayerSpec("attention", 2, c["num_kv_heads"], c["head_size"]),))
    cache = lv.PagedKVCache(spec, lv.PagedKVCacheConfig(num_blocks=c["num_blocks"], block_size=c["block_size"],
                                                        dtype=torch.float32, device=DEV))
    prefix = torch.tensor(c["prefix_keys"], dtype=torch.float32, device=DEV)
    cache.write("attention", prefix, prefix + c["prefix_value_offset"], torch.tensor(c["prefix_slots"], device=DEV))
    layout = lv.QueryLayout(tuple(c["parents"]))
    md = lv.PagedAttentionMetadata(block_tables=(tuple(c["block_table"]),), num_computed_tokens=(c["num_computed_tokens"],),
                                   query_layouts=(layout,), num_readonly_prefix_blocks=(c["num_readonly_prefix_blocks"],))
    qk = torch.tensor(c["query_keys"], dtype=torch.float32, device=DEV)
    cache.write("attention", qk, qk + c["query_value_offset"], md.slot_mapping(block_size=c["block_size"], device=DEV))
    moved = cache.compact(tuple(c["block_table"]), num_computed_tokens=c["num_computed_tokens"],
                          num_query_tokens=len(layout), num_reserved_query_tokens=len(layout),
                          retained_query_indices=tuple(c["retained"]),
                          num_readonly_prefix_blocks=c["num_readonly_prefix_blocks"])
    torch.cuda.synchronize()
    layer = cache.layer("attention")
    flat_k = layer.keys.view(-1, c["num_kv_heads"], c["head_size"])
    flat_v = layer.values.view(-1, c["num_kv_heads"], c["head_size"])
    assert torch.equal(layer.keys[1], prefix)
    assert torch.equal(flat_k[c["destination_slots"]], qk[c["retained"]])
    assert torch.equal(flat_v[c["destination_slots"]], qk[c["retained"]] + c["query_value_offset"])
    assert moved == c["expected_moved"]


@pytest.mark.parametrize("n_retained", [1, 5, 9, 16, 17, 40])
def test_compact_matches_oracle_across_layers(n_retained) -> None:
    _announce(f"compact n={n_retained}")
    rng = np.random.default_rng(n_retained)
    bs, nb, layers, computed = 16, 96, 3, 37
    q = max(n_retained + 3, 9)
    cache = _cache(hkv=2, d=128, bs=bs, nb=nb, dtype=torch.bfloat16, layers=layers, hq=12)
    table = tuple(int(b) for b in rng.permutation(nb)[: (computed + q + bs - 1) // bs])
    retained = tuple(int(i) for i in rng.permutation(q)[:n_retained])
    pools = [(_bits(cache.layer(f"l{i}").keys), _bits(cache.layer(f"l{i}").values)) for i in range(layers)]
    expect_moved = O.compact(pools, table, num_computed_tokens=computed, num_query_tokens=q,
                             num_reserved_query_tokens=q, retained_query_indices=retained, num_blocks=nb, block_size=bs)
    moved = cache.compact(table, num_computed_tokens=computed, num_query_tokens=q, num_reserved_query_tokens=q,
                          retained_query_indices=retained)
    torch.cuda.synchronize()
    assert moved == expect_moved
    for i, (kb, vb) in enumerate(pools):
        np.testing.assert_array_equal(_bits(cache.layer(f"l{i}").keys), kb)
        np.testing.assert_array_equal(_bits(cache.layer(f"l{i}").values), vb)


@pytest.mark.parametrize("after_create", [False, True])
@pytest.mark.parametrize("n_requests", [1, 3, 32])
def test_compact_many_matches_per_request_oracle(n_requests, after_create) -> None:
    # One launch for every request of a step: the same bytes as compacting the
    # requests one by one (oracle), and the same moved counts.  after_create:
    # the step's attention context has run over the same tables first.
    _announce(f"compact many x{n_requests} after_create={after_create}")
    rng = np.random.default_rng(100 + n_requests)
    bs, layers, computed, q = 16, 3, 29, 9
    per_req = (computed + q + bs - 1) // bs
    nb = per_req * n_requests + 5
    cache = _cache(hkv=2, d=128, bs=bs, nb=nb, dtype=torch.bfloat16, layers=layers, hq=12)
    perm = [int(x) for x in rng.permutation(nb)]
    pools = [(_bits(cache.layer(f"l{i}").keys), _bits(cache.layer(f"l{i}").values)) for i in range(layers)]
    requests, expect = [], []
    for r in range(n_requests):
        table = tuple(perm[r * per_req : (r + 1) * per_req])
        n_keep = int(rng.integers(1, q + 1))
        retained = tuple(sorted(int(i) for i in rng.permutation(q)[:n_keep]))
        args = dict(num_computed_tokens=computed, num_query_tokens=q, num_reserved_query_tokens=q,
                    retained_query_indices=retained)
        expect.append(O.compact(pools, table, num_blocks=nb, block_size=bs, **args))
        requests.append(dict(block_ids=table, **args))
    if after_create:
        md = lv.PagedAttentionMetadata(block_tables=tuple(r["block_ids"] for r in requests),
                                       num_computed_tokens=(computed,) * n_requests,
                                       query_layouts=(lv.linear_query_layout(q),) * n_requests)
        lv.HipPagedAttentionBackend().create(cache, md)
    moved = cache.compact_many(requests)
    torch.cuda.synchronize()
    assert moved == tuple(expect)
    for i, (kb, vb) in enumerate(pools):
        np.testing.assert_array_equal(_bits(cache.layer(f"l{i}").keys), kb)
        np.testing.assert_array_equal(_bits(cache.layer(f"l{i}").values), vb)


@pytest.mark.parametrize(
    "dtype,bs,n_requests,max_q,mixed",
    [
        (torch.bfloat16, 16, 16, 12, False),   # C5-shaped: accepted paths of 16 requests
        (torch.float16, 3, 5, 40, True),       # odd block size, layers of two row sizes
        (torch.float32, 16, 2, 64, False),     # a group at the length cap (4 batches of 16)
        (torch.bfloat16, 1, 40, 9, True),      # one-token blocks
    ],
)
def test_ordered_compact_is_one_pass_and_matches_the_oracle(dtype, bs, n_requests, max_q, mixed) -> None:
    # Strictly increasing retained indices over more pairs than ride in the
    # kernel arguments: compact_many takes the one-pass in-place kernel
    # (lvamd_kv_compact_ordered), and every byte of every layer equals the
    # oracle's per-request compact.
    from light_vllm_amd import native
    from light_vllm_amd.paged_cache import _compact_plan, ordered_groups

    _announce(f"ordered compact {dtype} bs={bs} x{n_requests} q<={max_q} mixed={mixed}")
    rng = np.random.default_rng(300 + n_requests * bs)
    shapes = [(2, 128), (4, 64), (1, 80)] if mixed else [(2, 128)] * 3
    spec = lv.ModelKVCacheSpec(tuple(lv.AttentionLayerSpec(f"l{i}", 8, hkv, d) for i, (hkv, d) in enumerate(shapes)))
    specs, num_blocks = [], 0
    for r in range(n_requests):
        computed, q = int(rng.integers(0, 50)), int(rng.integers(1, max_q + 1)) if r else max_q
        retained = tuple(sorted(int(x) for x in rng.permutation(q)[: int(rng.integers(1, q + 1))]))
        if r == 0:
            retained = tuple(range(1, q)) if q > 1 else (0,)  # the longest group moves q - 1 rows
        specs.append((computed, q, retained))
        num_blocks += (computed + q + bs - 1) // bs
    num_blocks += 3
    cache = lv.PagedKVCache(spec, lv.PagedKVCacheConfig(num_blocks=num_blocks, block_size=bs, dtype=dtype,
                                                        device=DEV))
    gen = torch.Generator(device=DEV).manual_seed(num_blocks)
    for i in range(len(shapes)):
        for pool in (cache.layer(f"l{i}").keys, cache.layer(f"l{i}").values):
            pool.copy_(torch.randn(pool.shape, generator=gen, device=DEV).to(dtype))
    perm = [int(x) for x in rng.permutation(num_blocks)]
    requests, off = [], 0
    for computed, q, retained in specs:
        need = (computed + q + bs - 1) // bs
        requests.append(dict(block_ids=tuple(perm[off : off + need]), num_computed_tokens=computed,
                             num_query_tokens=q, num_reserved_query_tokens=q, retained_query_indices=retained))
        off += need
    moved, src, dst = _compact_plan(cache.config, requests)
    assert src.size > native.load().lvamd_kv_compact_inline_pairs()
    assert ordered_groups(moved, src, dst) is not None, "this step must take the one-pass compact"
    pools = [(_bits(cache.layer(f"l{i}").keys), _bits(cache.layer(f"l{i}").values)) for i in range(len(shapes))]
    expect = []
    for req in requests:
        args = {k: v for k, v in req.items() if k != "block_ids"}
        expect.append(O.compact(pools, req["block_ids"], num_blocks=num_blocks, block_size=bs, **args))
    got_moved = cache.compact_many(requests)
    torch.cuda.synchronize()
    assert got_moved == tuple(expect)
    for i, (kb, vb) in enumerate(pools):
        np.testing.assert_array_equal(_bits(cache.layer(f"l{i}").keys), kb, err_msg=f"layer {i} keys")
        np.testing.assert_array_equal(_bits(cache.layer(f"l{i}").values), vb, err_msg=f"layer {i} values")


@pytest.mark.parametrize("layers,groups", [(5, 30), (8, 64)])
def test_ordered_compact_c_abi_matches_the_two_phase_compact(layers, groups) -> None:
    # Through the C ABI on identical pools: lvamd_kv_compact_ordered and
    # lvamd_kv_compact give the same bytes for a grouped, ordered pair list
    # (groups of 1 to 40 pairs; each group reads rows at or after the ones it
    # writes), and zero groups is a no-op.  Chunk widths: 5 layers x 30
    # groups is narrowed to 8-byte chunks (fewer than 64 workgroups of 16-byte
    # items); 8 layers x 64 groups (32,768 items of 16 bytes) keeps 16-byte
    # chunks, whose batches hold 8 pairs, so longer groups take several.
    from light_vllm_amd import native

    _announce(f"ordered compact vs two-phase compact (C ABI), {layers} layers x {groups} groups")
    lib = native.load()
    stream = torch.cuda.current_stream(DEV).cuda_stream
    slots, row = 8192, 2 * 128 * 2
    gen = torch.Generator(device=DEV).manual_seed(3)
    a = [torch.randn((slots, 2, 128), generator=gen, device=DEV).to(torch.bfloat16) for _ in range(2 * layers)]
    b = [t.clone() for t in a]
    rng = np.random.default_rng(4)
    src, dst, starts, base = [], [], [0], 0
    sizes = rng.integers(1, 41, size=groups)
    assert (sizes > 8).any() and (sizes <= 8).any()
    for size in sizes:
        keep = np.sort(rng.choice(np.arange(1, 2 * size), size=size, replace=False))
        src += [base + int(k) for k in keep]
        dst += [base + i for i in range(size)]
        starts.append(starts[-1] + int(size))
        base += 2 * int(size) + 5
    src_t = torch.tensor(src, dtype=torch.int64, device=DEV)
    dst_t = torch.tensor(dst, dtype=torch.int64, device=DEV)
    starts_t = torch.tensor(starts, dtype=torch.int64, device=DEV)

    def tables(pools):
        k = torch.tensor([t.data_ptr() for t in pools[0::2]], dtype=torch.int64, device=DEV)
        v = torch.tensor([t.data_ptr() for t in pools[1::2]], dtype=torch.int64, device=DEV)
        return k, v

    (ka, va), (kb, vb) = tables(a), tables(b)
    before = [t.view(torch.int16).cpu().numpy().reshape(slots, -1) for t in a]
    n = len(src)
    ws_bytes = lib.lvamd_kv_compact_workspace_size(n, layers, row)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    native.check(lib.lvamd_kv_compact(ka.data_ptr(), va.data_ptr(), layers, row, src_t.data_ptr(), dst_t.data_ptr(),
                                      n, ws.data_ptr(), ws_bytes, stream), "lvamd_kv_compact")
    native.check(lib.lvamd_kv_compact_ordered(kb.data_ptr(), vb.data_ptr(), layers, row, src_t.data_ptr(),
                                              dst_t.data_ptr(), starts_t.data_ptr(), len(starts) - 1, stream),
                 "lvamd_kv_compact_ordered")
    native.check(lib.lvamd_kv_compact_ordered(kb.data_ptr(), vb.data_ptr(), layers, row, src_t.data_ptr(),
                                              dst_t.data_ptr(), starts_t.data_ptr(), 0, stream),
                 "lvamd_kv_compact_ordered")
    torch.cuda.synchronize()
    for i, (x, y, rows) in enumerate(zip(a, b, before)):
        expect = rows.copy()
        expect[dst] = rows[src]  # every source read before any destination is written
        np.testing.assert_array_equal(y.view(torch.int16).cpu().numpy().reshape(slots, -1), expect,
                                      err_msg=f"pool {i} vs closed form")
        assert torch.equal(x.view(torch.int16), y.view(torch.int16)), f"pool {i} vs two-phase compact"


def test_compact_many_rejects_a_shared_destination() -> None:
    cache = _cache(hkv=2, d=64, bs=2, nb=8, dtype=torch.float32)
    req = dict(block_ids=(0, 1), num_computed_tokens=1, num_query_tokens=2, num_reserved_query_tokens=2,
               retained_query_indices=(1,))
    with pytest.raises(lv.KVCacheError, match="same slot"):
        cache.compact_many([req, req])


def test_compact_identity_path_writes_nothing_and_returns_zero() -> None:
    cache = _cache(hkv=2, d=64, bs=4, nb=8, dtype=torch.float32)
    before = _bits(cache.layer("l0").keys)
    assert cache.compact((3, 1), num_computed_tokens=2, num_query_tokens=3, num_reserved_query_tokens=3,
                         retained_query_indices=(0, 1, 2)) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(cache.layer("l0").keys), before)


def test_compact_validation_errors() -> None:
    cache = _cache(hkv=2, d=64, bs=2, nb=8, dtype=torch.float32)
    with pytest.raises(lv.KVCacheError, match="exceeds the paged KV tail"):
        cache.compact((0, 1), num_computed_tokens=1, num_query_tokens=2, num_reserved_query_tokens=2,
                      retained_query_indices=(2,))
    with pytest.raises(ValueError, match="unique"):
        cache.compact((0, 1), num_computed_tokens=1, num_query_tokens=2, num_reserved_query_tokens=2,
                      retained_query_indices=(1, 1))
    with pytest.raises(lv.KVCacheError, match="exactly cover"):
        cache.compact((0,), num_computed_tokens=1, num_query_tokens=2, num_reserved_query_tokens=2,
                      retained_query_indices=(1,))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_block_copy_matches_closed_form(dtype) -> None:
    _announce(f"block copy {dtype}")
    rng = np.random.default_rng(5)
    nb, layers = 200, 4
    cache = _cache(hkv=2, d=128, bs=16, nb=nb, dtype=dtype, layers=layers, hq=12)
    perm = [int(x) for x in rng.permutation(nb)]
    src, dst = perm[:32], perm[32:64]
    pools = [(_bits(cache.layer(f"l{i}").keys), _bits(cache.layer(f"l{i}").values)) for i in range(layers)]
    O.block_copy(pools, src, dst)
    cache.copy_blocks(src, dst)
    torch.cuda.synchronize()
    for i, (kb, vb) in enumerate(pools):
        np.testing.assert_array_equal(_bits(cache.layer(f"l{i}").keys), kb)
        np.testing.assert_array_equal(_bits(cache.layer(f"l{i}").values), vb)


def test_block_copy_rejects_overlap_and_duplicates() -> None:
    cache = _cache(hkv=2, d=64, bs=4, nb=8, dtype=torch.float32)
    with pytest.raises(lv.KVCacheError, match="disjoint"):
        cache.copy_blocks([1, 2], [2, 3])
    with pytest.raises(lv.KVCacheError, match="twice"):
        cache.copy_blocks([1, 2], [4, 4])
    with pytest.raises(lv.KVCacheError, match="invalid physical block"):
        cache.copy_blocks([1], [8])


@pytest.mark.parametrize("nbytes, workgroups", [(16, 1), (4096, 3), ((1 << 20) + 48, 512), (64 << 20, 1024)])
def test_read_probe_reads_every_chunk_once(nbytes, workgroups) -> None:
    """The bandwidth probe bench.py times reads each 16-byte chunk exactly
    once: the XOR of its per-lane words equals the XOR of the buffer."""

    from light_vllm_amd import native

    _announce(f"read probe {nbytes} B, {workgroups} workgroups")
    rng = np.random.default_rng(nbytes)
    words = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint64).astype(np.uint32)
    buf = torch.from_numpy(words.view(np.int32)).to(DEV)
    sink = torch.empty(workgroups * 64, dtype=torch.int32, device=DEV)
    lib = native.load()
    stream = torch.cuda.current_stream(DEV).cuda_stream
    native.check(lib.lvamd_hbm_read_probe(buf.data_ptr(), nbytes, sink.data_ptr(), workgroups, stream),
                 "lvamd_hbm_read_probe")
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(words)
    # A size that is not a multiple of 16 is refused (LVAMD_ERR_INVALID_ARGUMENT).
    assert lib.lvamd_hbm_read_probe(buf.data_ptr(), 8, sink.data_ptr(), workgroups, stream) == -1


def test_cache_built_from_the_capacity_planners_config() -> None:
    # light-vllm sizes the pool with CudaMemoryKVCachePlanner (paged_cache.py:
    # 69-114): free device memory x a fraction, divided by the bytes of one
    # block over all layers, in a PagedKVCacheConfig of its own class.  That
    # config builds this package's cache unchanged (its fields are read, not
    # its class), the pools hold exactly the planned bytes, and decode runs on
    # a cache so sized.
    _announce("cache from the capacity planner's config")
    from dataclasses import dataclass

    @dataclass(frozen=True)
    class PlannerConfig:  # the reference config's fields, another class
        num_blocks: int
        block_size: int
        dtype: torch.dtype
        device: torch.device

    layers = [(4, 128)] * 3
    spec = lv.ModelKVCacheSpec(tuple(lv.AttentionLayerSpec(f"l{i}", 28, hkv, d) for i, (hkv, d) in enumerate(layers)))
    free, _ = torch.cuda.mem_get_info(DEV)
    fraction = min(0.004, (1 << 30) / free)  # a small slice of the free memory
    num_blocks = O.planned_num_blocks(free, fraction, layers, block_size=16, element_size=2)
    assert num_blocks > 0
    config = PlannerConfig(num_blocks=num_blocks, block_size=16, dtype=torch.bfloat16, device=DEV)
    cache = lv.PagedKVCache(spec, config)
    pool_bytes = sum(cache.layer(f"l{i}").keys.nbytes + cache.layer(f"l{i}").values.nbytes for i in range(3))
    per_block = O.kv_cache_bytes_per_block(layers, block_size=16, element_size=2)
    assert pool_bytes == num_blocks * per_block <= int(free * fraction)
    assert cache.config is config
    computed = [100, 700]
    need = [(c + 1 + 15) // 16 for c in computed]
    tables = (tuple(range(need[0])), tuple(range(num_blocks - need[1], num_blocks)))
    md = lv.PagedAttentionMetadata(block_tables=tables, num_computed_tokens=tuple(computed),
                                   query_layouts=(lv.linear_query_layout(1), lv.linear_query_layout(1)))
    gen = torch.Generator(device=DEV).manual_seed(5)
    q = torch.randn((2, 28, 128), generator=gen, device=DEV).to(torch.bfloat16)
    k = torch.randn((2, 4, 128), generator=gen, device=DEV).to(torch.bfloat16)
    layer = cache.layer("l0")
    for pool in (layer.keys, layer.values):
        pool.zero_()
    out = lv.HipPagedAttentionBackend().create(cache, md).forward("l0", q, k, k, scale=0.1)
    torch.cuda.synchronize()
    # Zero history: each query sees its own key among zero keys, so the
    # output is the softmax-weighted mean of zero rows and its own value.
    scores = (q.float() * 0.1 * k.float().repeat_interleave(7, dim=1)).sum(-1)  # [2, 28]
    weight = torch.exp(scores) / (torch.exp(scores) + torch.tensor(computed, device=DEV)[:, None])
    expect = weight[..., None] * k.float().repeat_interleave(7, dim=1)
    assert (out.float() - expect).abs().max().item() <= 2e-2
