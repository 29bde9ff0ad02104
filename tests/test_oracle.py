"""Pins the CPU oracle before it is trusted as the GPU kernels' checker.

* Known answers transcribed from light-vllm's own tests (tests/golden/).
* Closed forms for the copies (moved rows byte-equal, every other byte unchanged).
* The online-softmax restatement against an independent fp64 dense softmax,
  plus closed forms (one visible key, identical keys).
* Planted mistakes: single-line edits of the oracle's own source (a GQA index,
  a dropped rescale term, a sign, an off-by-one block) must fail these checks.
"""

from __future__ import annotations

import inspect
import json
import textwrap
from pathlib import Path

import numpy as np
import pytest

from oracle import paged_kv_oracle as O

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


# ----------------------------------------------------------------------------- metadata
@pytest.mark.parametrize("case", GOLDEN["slot_mapping"], ids=lambda c: c["source"][:40])
def test_slot_mapping_known_answers(case) -> None:
    got = O.slot_mapping(
        case["block_tables"], case["num_computed_tokens"], case["query_lengths"], case["reserved"], case["block_size"]
    )
    assert got.tolist() == case["expected"]


@pytest.mark.parametrize("case", GOLDEN["validation_errors"], ids=lambda c: c["source"][-30:])
def test_validation_known_errors(case) -> None:
    n = len(case["block_tables"])
    readonly = case.get("readonly", [0] * n)
    with pytest.raises(O.OracleKVCacheError, match=case["match"]):
        O.validate_block_tables(
            case["block_tables"], case["num_computed_tokens"], case["query_lengths"], readonly,
            num_blocks=case["num_blocks"], block_size=case["block_size"],
        )


def test_validation_accepts_shared_readonly_prefix_and_lookahead() -> None:
    c = GOLDEN["valid_shared_prefix"]
    O.validate_block_tables(
        c["block_tables"], c["num_computed_tokens"], c["query_lengths"], c["readonly"],
        num_blocks=c["num_blocks"], block_size=c["block_size"],
    )
    look = GOLDEN["slot_mapping"][1]
    O.validate_block_tables(
        look["block_tables"], look["num_computed_tokens"], look["reserved"], [0],
        num_blocks=look["num_blocks"], block_size=look["block_size"],
    )


def test_visibility_packing_known_answer() -> None:
    c = GOLDEN["visibility_packing"]
    flat, starts = O.visibility_tensor([tuple(p) for p in c["layouts"]])
    assert flat.tolist() == c["visibility"]
    assert starts.tolist() == c["visibility_start"]
    assert O.request_indices([len(p) for p in c["layouts"]]).tolist() == c["request_indices"]


def test_query_layout_known_answers() -> None:
    c = GOLDEN["query_layout"]
    parents = tuple(c["parents"])
    assert list(O.semantic_positions(parents, c["prefix_length"])) == c["positions"]
    assert O.query_visibility(parents).tolist() == c["visibility"]
    d = c["append_draft"]
    assert list(O.append_draft_parents(d["num_inputs"], tuple(d["draft_parents"]))) == d["expected"]
    lin = GOLDEN["linear_detection"]
    assert all(O.is_linear(tuple(p)) for p in lin["linear"])
    assert not any(O.is_linear(tuple(p)) for p in lin["tree"])


def test_visible_positions_known_answer() -> None:
    c = GOLDEN["visible_positions"]
    assert O.visible_positions(c["num_computed_tokens"], tuple(c["parents"])) == c["expected"]


# ----------------------------------------------------------------------------- KV movement
def _compact_golden_pool():
    c = GOLDEN["compact"]
    shape = (c["num_blocks"], c["block_size"], c["num_kv_heads"], c["head_size"])
    kpool = np.full(shape, -1.0, dtype=np.float32)
    vpool = np.full(shape, -1.0, dtype=np.float32)
    prefix = np.asarray(c["prefix_keys"], dtype=np.float32)
    O.append(kpool, vpool, prefix, prefix + c["prefix_value_offset"], np.asarray(c["prefix_slots"]))
    parents = tuple(c["parents"])
    slots = O.slot_mapping([c["block_table"]], [c["num_computed_tokens"]], [len(parents)], [len(parents)], c["block_size"])
    qk = np.asarray(c["query_keys"], dtype=np.float32)
    O.append(kpool, vpool, qk, qk + c["query_value_offset"], slots)
    return c, kpool, vpool, prefix, qk


def test_compact_known_answer() -> None:
    c, kpool, vpool, prefix, qk = _compact_golden_pool()
    moved = O.compact(
        [(kpool, vpool)], tuple(c["block_table"]),
        num_computed_tokens=c["num_computed_tokens"], num_query_tokens=len(c["parents"]),
        num_reserved_query_tokens=len(c["parents"]), retained_query_indices=tuple(c["retained"]),
        num_readonly_prefix_blocks=c["num_readonly_prefix_blocks"],
        num_blocks=c["num_blocks"], block_size=c["block_size"],
    )
    flat_k = kpool.reshape(-1, c["num_kv_heads"], c["head_size"])
    flat_v = vpool.reshape(-1, c["num_kv_heads"], c["head_size"])
    np.testing.assert_array_equal(kpool[1], prefix)
    np.testing.assert_array_equal(flat_k[c["destination_slots"]], qk[c["retained"]])
    np.testing.assert_array_equal(flat_v[c["destination_slots"]], qk[c["retained"]] + c["query_value_offset"])
    assert moved == c["expected_moved"]


def test_contiguous_compact_known_answer_on_a_paged_pool() -> None:
    # The contiguous analogue (tests/test_kv_cache.py:553-573) on a block_size-1 pool
    # whose table is the identity: the formal tail keeps retained entries in order.
    c = GOLDEN["contiguous_compact"]
    seq = np.asarray(c["sequence"], dtype=np.float32).reshape(-1, 1, 1, 1)
    kpool = seq.copy()
    vpool = seq.copy()
    n_query = len(c["sequence"]) - c["num_computed_tokens"]
    O.compact(
        [(kpool, vpool)], tuple(range(len(c["sequence"]))),
        num_computed_tokens=c["num_computed_tokens"], num_query_tokens=n_query, num_reserved_query_tokens=n_query,
        retained_query_indices=tuple(c["retained"]), num_blocks=len(c["sequence"]), block_size=1,
    )
    assert kpool.reshape(-1)[: len(c["expected"])].tolist() == c["expected"]


def test_compact_identity_path_writes_nothing() -> None:
    pool = np.arange(4 * 2 * 1 * 2, dtype=np.float32).reshape(4, 2, 1, 2)
    before = pool.copy()
    moved = O.compact(
        [(pool, pool.copy())], (0, 1), num_computed_tokens=1, num_query_tokens=3, num_reserved_query_tokens=3,
        retained_query_indices=(0, 1), num_blocks=4, block_size=2,
    )
    assert moved == 0
    np.testing.assert_array_equal(pool, before)


def _compact_sequential(pools, src, dst):
    """Planted mistake: scatter pair by pair (no gather-before-scatter)."""
    for kp, vp in pools:
        for pool in (kp, vp):
            flat = pool.reshape(-1, *pool.shape[2:])
            for s, d in zip(src, dst):
                flat[d] = flat[s]


@pytest.mark.parametrize("seed", range(6))
def test_compact_closed_form_on_random_overlapping_paths(seed) -> None:
    rng = np.random.default_rng(seed)
    bs, nb, computed, q = 4, 16, 5, 9
    table = tuple(int(b) for b in rng.permutation(nb)[: (computed + q + bs - 1) // bs])
    retained = tuple(int(i) for i in rng.permutation(q)[: rng.integers(2, q)])
    pools = [(rng.standard_normal((nb, bs, 2, 8)).astype(np.float32),
              rng.standard_normal((nb, bs, 2, 8)).astype(np.float32)) for _ in range(3)]
    originals = [(k.copy(), v.copy()) for k, v in pools]
    O.compact(pools, table, num_computed_tokens=computed, num_query_tokens=q, num_reserved_query_tokens=q,
              retained_query_indices=retained, num_blocks=nb, block_size=bs)

    def slot(pos):
        return table[pos // bs] * bs + pos % bs

    src = [slot(computed + i) for i in retained]
    dst = [slot(computed + i) for i in range(len(retained))]
    for (k, v), (k0, v0) in zip(pools, originals):
        for now, before in ((k, k0), (v, v0)):
            expect = before.reshape(nb * bs, 2, 8).copy()
            expect[dst] = before.reshape(nb * bs, 2, 8)[src]
            np.testing.assert_array_equal(now.reshape(nb * bs, 2, 8), expect)


def test_planted_sequential_compact_fails_closed_form() -> None:
    # retained (2, 0): target 0 <- source 2, then target 1 <- source 0 (already overwritten).
    pool_k = np.arange(8, dtype=np.float32).reshape(8, 1, 1, 1)
    pools = [(pool_k.copy(), pool_k.copy())]
    table = (0, 1, 2)
    _compact_sequential(pools, [2, 0], [0, 1])
    expect = pool_k.reshape(-1).copy()
    expect[[0, 1]] = pool_k.reshape(-1)[[2, 0]]
    assert not np.array_equal(pools[0][0].reshape(-1), expect)
    correct = [(pool_k.copy(), pool_k.copy())]
    O.compact(correct, table, num_computed_tokens=0, num_query_tokens=3, num_reserved_query_tokens=3,
              retained_query_indices=(2, 0), num_blocks=8, block_size=1)
    np.testing.assert_array_equal(correct[0][0].reshape(-1), expect)


def test_append_closed_form_touches_only_written_slots() -> None:
    rng = np.random.default_rng(7)
    kpool = rng.integers(0, 2**16, size=(8, 4, 2, 16), dtype=np.uint16)
    vpool = rng.integers(0, 2**16, size=(8, 4, 2, 16), dtype=np.uint16)
    k0, v0 = kpool.copy(), vpool.copy()
    key = rng.integers(0, 2**16, size=(5, 2, 16), dtype=np.uint16)
    value = rng.integers(0, 2**16, size=(5, 2, 16), dtype=np.uint16)
    slots = np.array([3, 17, -1, 30, 0])
    O.append(kpool, vpool, key, value, slots)
    fk, fv = kpool.reshape(32, 2, 16), vpool.reshape(32, 2, 16)
    for t, s in enumerate(slots):
        if s >= 0:
            np.testing.assert_array_equal(fk[s], key[t])
            np.testing.assert_array_equal(fv[s], value[t])
    untouched = np.setdiff1d(np.arange(32), slots[slots >= 0])
    np.testing.assert_array_equal(fk[untouched], k0.reshape(32, 2, 16)[untouched])
    np.testing.assert_array_equal(fv[untouched], v0.reshape(32, 2, 16)[untouched])


def test_block_copy_closed_form() -> None:
    rng = np.random.default_rng(3)
    pools = [(rng.standard_normal((6, 4, 2, 8)), rng.standard_normal((6, 4, 2, 8))) for _ in range(2)]
    before = [(k.copy(), v.copy()) for k, v in pools]
    O.block_copy(pools, [0, 2], [5, 1])
    for (k, v), (k0, v0) in zip(pools, before):
        for now, old in ((k, k0), (v, v0)):
            np.testing.assert_array_equal(now[5], old[0])
            np.testing.assert_array_equal(now[1], old[2])
            np.testing.assert_array_equal(now[[0, 2, 3, 4]], old[[0, 2, 3, 4]])


# ----------------------------------------------------------------------------- attention
def random_case(rng, *, hq, hkv, d, bs, computed, layouts, num_blocks=None, shared_prefix_blocks=0):
    """Random pools with every referenced position written, disjoint tables."""

    q_lens = [len(p) for p in layouts]
    need = [(c + q + bs - 1) // bs for c, q in zip(computed, q_lens)]
    total = shared_prefix_blocks + sum(n - shared_prefix_blocks for n in need)
    nb = num_blocks or total + 3
    perm = [int(x) for x in rng.permutation(nb)]
    shared = perm[:shared_prefix_blocks]
    rest = perm[shared_prefix_blocks:]
    tables = []
    for n in need:
        tables.append(tuple(shared + rest[: n - shared_prefix_blocks]))
        rest = rest[n - shared_prefix_blocks:]
    kpool = rng.standard_normal((nb, bs, hkv, d)).astype(np.float32)
    vpool = rng.standard_normal((nb, bs, hkv, d)).astype(np.float32)
    t = sum(q_lens)
    query = rng.standard_normal((t, hq, d)).astype(np.float32)
    return query, kpool, vpool, tables


CASES = [
    dict(hq=2, hkv=2, d=4, bs=2, computed=[0], layouts=[(-1, 0, 0, 2)]),                 # tree, reference 84-118
    dict(hq=2, hkv=2, d=4, bs=2, computed=[0, 0], layouts=[(-1, 0, 1), (-1, 0)]),        # multi-request prefill
    dict(hq=4, hkv=2, d=4, bs=2, computed=[0], layouts=[(-1, 0, 1)]),                     # GQA, reference 287-309
    dict(hq=14, hkv=2, d=64, bs=16, computed=[37, 128, 200, 511], layouts=[(-1,)] * 4),  # C1 decode
    dict(hq=28, hkv=4, d=128, bs=16, computed=[130], layouts=[(-1,)]),                    # long history
    dict(hq=12, hkv=2, d=32, bs=4, computed=[9, 3], layouts=[(-1, 0, 0, 1, 2, 2, 5, 6, 0), (-1, 0, 1)]),
]


@pytest.mark.parametrize("case", CASES, ids=range(len(CASES)))
def test_online_oracle_matches_fp64_dense(case) -> None:
    rng = np.random.default_rng(11)
    query, kpool, vpool, tables = random_case(rng, **case)
    scale = 1.0 / np.sqrt(case["d"])
    online = O.paged_attention(query, kpool, vpool, tables, case["computed"], case["layouts"], scale=scale)
    dense = O.dense_attention(query, kpool, vpool, tables, case["computed"], case["layouts"], scale=scale)
    np.testing.assert_allclose(online, dense, atol=2e-6, rtol=0)


def test_shared_readonly_prefix_matches_dense() -> None:
    rng = np.random.default_rng(5)
    case = dict(hq=4, hkv=2, d=16, bs=4, computed=[8, 8], layouts=[(-1,), (-1, 0)], shared_prefix_blocks=2)
    query, kpool, vpool, tables = random_case(rng, **case)
    assert tables[0][:2] == tables[1][:2]
    online = O.paged_attention(query, kpool, vpool, tables, case["computed"], case["layouts"], scale=0.25)
    dense = O.dense_attention(query, kpool, vpool, tables, case["computed"], case["layouts"], scale=0.25)
    np.testing.assert_allclose(online, dense, atol=2e-6, rtol=0)


def test_single_visible_key_returns_its_value() -> None:
    rng = np.random.default_rng(2)
    query, kpool, vpool, tables = random_case(rng, hq=6, hkv=2, d=8, bs=4, computed=[0, 0], layouts=[(-1,), (-1,)])
    out = O.paged_attention(query, kpool, vpool, tables, [0, 0], [(-1,), (-1,)], scale=0.3)
    for r, table in enumerate(tables):
        v = vpool[table[0], 0]  # position 0 of request r, [Hkv, D]
        np.testing.assert_array_equal(out[r], np.repeat(v, 3, axis=0))


def test_identical_keys_give_the_mean_of_values() -> None:
    rng = np.random.default_rng(4)
    query, kpool, vpool, tables = random_case(rng, hq=4, hkv=1, d=8, bs=4, computed=[10], layouts=[(-1,)])
    kpool[:] = kpool[0, 0]
    out = O.paged_attention(query, kpool, vpool, tables, [10], [(-1,)], scale=0.5)
    pos = np.arange(11)
    vals = vpool[np.asarray(tables[0])[pos // 4], pos % 4]  # [11, 1, D]
    np.testing.assert_allclose(out[0], np.repeat(vals.mean(axis=0), 4, axis=0), atol=1e-6)


MUTATIONS = {
    "gqa_index": ("keys = np.repeat(keys, repeats, axis=1)", "keys = np.tile(keys, (1, repeats, 1))"),
    "dropped_rescale": ("acc = acc * prev_scale[:, None] +", "acc = acc +"),
    "wrong_sign": ("* scale32", "* -scale32"),
    "block_index": ("blk = table[logical]", "blk = table[max(logical - 1, 0)]"),
}


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_planted_oracle_mistakes_fail_the_dense_check(name) -> None:
    old, new = MUTATIONS[name]
    source = textwrap.dedent(inspect.getsource(O.paged_attention))
    assert old in source, f"mutation anchor for {name} not found"
    namespace = dict(vars(O))
    exec(compile(source.replace(old, new), "<mutant>", "exec"), namespace)
    mutant = namespace["paged_attention"]
    rng = np.random.default_rng(21)
    case = dict(hq=8, hkv=2, d=16, bs=4, computed=[13, 6], layouts=[(-1,), (-1, 0, 0)])
    query, kpool, vpool, tables = random_case(rng, **case)
    dense = O.dense_attention(query, kpool, vpool, tables, case["computed"], case["layouts"], scale=0.25)
    good = O.paged_attention(query, kpool, vpool, tables, case["computed"], case["layouts"], scale=0.25)
    bad = mutant(query, kpool, vpool, tables, case["computed"], case["layouts"], scale=0.25)
    assert np.abs(good - dense).max() < 2e-6
    assert np.abs(bad - dense).max() > 1e-2


# --------------------------------------------------------------------------- rotary
TORCH_DTYPES = {"bf16": "bfloat16", "f16": "float16", "f32": "float32"}


def _rotary_inputs(rng, dtype, tokens=5, heads=3, d=16, theta=10000.0):
    import torch

    tdt = getattr(torch, TORCH_DTYPES[dtype])
    x = torch.randn(tokens, heads, d, generator=torch.Generator().manual_seed(int(rng.integers(1 << 30)))).to(tdt)
    pos = torch.as_tensor(rng.integers(0, 40000, size=tokens), dtype=torch.float32)
    freqs = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    angles = torch.outer(pos, freqs)
    emb = torch.cat((angles, angles), dim=-1)
    return x, emb.cos().to(tdt), emb.sin().to(tdt)


def _as_bits(t):
    import torch

    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("seed", range(4))
def test_rotary_matches_torch_dtype_arithmetic(dtype, seed) -> None:
    """The oracle's rounding emulation equals torch's own CPU arithmetic in the
    tensor dtype on the reference's expression (what the reference runs
    without Triton), bit for bit."""

    import torch

    rng = np.random.default_rng(seed)
    x, cos, sin = _rotary_inputs(rng, dtype, d=[16, 64, 128, 80][seed])
    if seed == 3:
        x = x * 300.0  # large magnitudes: the float32 sum can round twice
    first, second = x.chunk(2, dim=-1)
    expected = x * cos.unsqueeze(1) + torch.cat((-second, first), dim=-1) * sin.unsqueeze(1)
    got = O.rotary_half(_as_bits(x), _as_bits(cos), _as_bits(sin), dtype)
    np.testing.assert_array_equal(got, _as_bits(expected))


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_rotary_closed_forms(dtype) -> None:
    """cos 1 / sin 0 is the identity; cos 0 / sin 1 is the half swap with the
    first half negated; cos -1 / sin 0 negates."""

    import torch

    rng = np.random.default_rng(7)
    x, cos, sin = _rotary_inputs(rng, dtype)
    xb = _as_bits(x)
    one, zero = torch.ones_like(cos), torch.zeros_like(cos)
    np.testing.assert_array_equal(O.rotary_half(xb, _as_bits(one), _as_bits(zero), dtype), xb)
    swapped = torch.cat((-x[..., 8:], x[..., :8]), dim=-1)
    np.testing.assert_array_equal(O.rotary_half(xb, _as_bits(zero), _as_bits(one), dtype), _as_bits(swapped))
    np.testing.assert_array_equal(O.rotary_half(xb, _as_bits(-one), _as_bits(zero), dtype), _as_bits(-x))


def test_rotary_preserves_pair_norms() -> None:
    """Each (d, d + D/2) pair is rotated by one angle: its norm is kept (fp32)."""

    rng = np.random.default_rng(9)
    x, cos, sin = _rotary_inputs(rng, "f32", tokens=7, heads=2, d=32)
    out = O.rotary_half(_as_bits(x), _as_bits(cos), _as_bits(sin), "f32").astype(np.float64)
    xin = x.numpy().astype(np.float64)
    norm_in = xin[..., :16] ** 2 + xin[..., 16:] ** 2
    norm_out = out[..., :16] ** 2 + out[..., 16:] ** 2
    np.testing.assert_allclose(norm_out, norm_in, rtol=2e-6, atol=1e-9)


ROTARY_MUTATIONS = {
    "sign": ("(-xf[..., half:], xf[..., :half])", "(xf[..., half:], xf[..., :half])"),
    "pairing": ("np.concatenate((-xf[..., half:], xf[..., :half]), axis=-1)",
                "np.stack((-xf[..., 1::2], xf[..., ::2]), axis=-1).reshape(xf.shape)"),
    "single_rounding": ("first + second", "xf * c + rotated * s"),
}


@pytest.mark.parametrize("name", sorted(ROTARY_MUTATIONS))
def test_planted_rotary_mistakes_fail(name) -> None:
    import torch

    old, new = ROTARY_MUTATIONS[name]
    source = textwrap.dedent(inspect.getsource(O.rotary_half))
    assert old in source, f"mutation anchor for {name} not found"
    namespace = dict(vars(O))
    exec(compile(source.replace(old, new), "<mutant>", "exec"), namespace)
    mutant = namespace["rotary_half"]
    rng = np.random.default_rng(11)
    x, cos, sin = _rotary_inputs(rng, "bf16", tokens=16, heads=4, d=64)
    first, second = x.chunk(2, dim=-1)
    expected = _as_bits(x * cos.unsqueeze(1) + torch.cat((-second, first), dim=-1) * sin.unsqueeze(1))
    good = O.rotary_half(_as_bits(x), _as_bits(cos), _as_bits(sin), "bf16")
    bad = mutant(_as_bits(x), _as_bits(cos), _as_bits(sin), "bf16")
    np.testing.assert_array_equal(good, expected)
    assert (bad != expected).any()


# ------------------------------------------------------ capacity planner arithmetic
def test_bytes_per_block_known_answers() -> None:
    # Qwen2.5-7B: 28 layers x K and V x 4 kv heads x 128 dims x 16 tokens x 2 bytes.
    assert O.kv_cache_bytes_per_block([(4, 128)] * 28, block_size=16, element_size=2) == 917_504
    # Qwen2.5-1.5B: 28 x 2 x 2 x 128 x 16 x 2; Qwen2.5-0.5B in fp32: 24 x 2 x 2 x 64 x 16 x 4.
    assert O.kv_cache_bytes_per_block([(2, 128)] * 28, block_size=16, element_size=2) == 458_752
    assert O.kv_cache_bytes_per_block([(2, 64)] * 24, block_size=16, element_size=4) == 393_216
    # Layers of different kv shapes add up.
    assert O.kv_cache_bytes_per_block([(4, 128), (2, 64)], block_size=1, element_size=2) == 2 * (512 + 128) * 2


@pytest.mark.parametrize("seed", range(5))
def test_planned_blocks_are_the_most_that_fit_the_budget(seed) -> None:
    # Brute force: blocks added one by one until the next one would exceed
    # int(free * fraction) bytes.
    rng = np.random.default_rng(seed)
    layers = [(int(rng.choice([1, 2, 4, 8])), int(rng.choice([64, 80, 128]))) for _ in range(int(rng.integers(1, 6)))]
    bs, es = int(rng.choice([1, 16, 32])), int(rng.choice([2, 4]))
    free = int(rng.integers(1 << 20, 1 << 28))
    fraction = float(rng.uniform(0.05, 1.0))
    per_block = O.kv_cache_bytes_per_block(layers, block_size=bs, element_size=es)
    n = 0
    while (n + 1) * per_block <= int(free * fraction):
        n += 1
    assert O.planned_num_blocks(free, fraction, layers, block_size=bs, element_size=es) == n
    assert O.planned_num_blocks(per_block - 1, 1.0, layers, block_size=bs, element_size=es) == 0


def test_package_bytes_per_block_follow_the_planner() -> None:
    # The backend's own figure (PagedKVCache allocates exactly this per block)
    # equals the planner's, so a planner budget maps to the same block count.
    import light_vllm_amd as lv
    import torch

    spec = lv.ModelKVCacheSpec((lv.AttentionLayerSpec("a", 28, 4, 128), lv.AttentionLayerSpec("b", 12, 2, 64)))
    for dtype, es in ((torch.bfloat16, 2), (torch.float32, 4)):
        got = lv.paged_cache.kv_cache_bytes_per_block(spec, block_size=16, dtype=dtype)
        assert got == O.kv_cache_bytes_per_block([(4, 128), (2, 64)], block_size=16, element_size=es)
