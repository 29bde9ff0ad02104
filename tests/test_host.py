"""CPU tests of the host side: the restated metadata/layout/validation against
the reference's known answers and the oracle, the step planner's device
metadata, and the C-ABI library's exports (loaded, no kernel launched)."""

from __future__ import annotations

import math

import ctypes
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import light_vllm_amd as lv
from light_vllm_amd import native
from light_vllm_amd.plan import LayerShapes, Staging, StepPlan
from oracle import paged_kv_oracle as O

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())
CPU = torch.device("cpu")


def _layouts(*lengths):
    return tuple(lv.linear_query_layout(n) for n in lengths)


def _metadata(case):
    n = len(case["block_tables"])
    return lv.PagedAttentionMetadata(
        block_tables=tuple(tuple(t) for t in case["block_tables"]),
        num_computed_tokens=tuple(case["num_computed_tokens"]),
        query_layouts=_layouts(*case["query_lengths"]),
        num_reserved_query_tokens=tuple(case.get("reserved", case["query_lengths"])),
        num_readonly_prefix_blocks=tuple(case.get("readonly", [0] * n)),
    )


@pytest.mark.parametrize("case", GOLDEN["slot_mapping"], ids=lambda c: c["source"][:40])
def test_metadata_slot_mapping_known_answers(case) -> None:
    assert _metadata(case).slot_mapping(block_size=case["block_size"], device=CPU).tolist() == case["expected"]


@pytest.mark.parametrize("case", GOLDEN["validation_errors"], ids=lambda c: c["source"][-30:])
def test_metadata_validation_known_errors(case) -> None:
    with pytest.raises(lv.KVCacheError, match=case["match"]):
        _metadata(case).validate_block_tables(num_blocks=case["num_blocks"], block_size=case["block_size"])


def test_metadata_visibility_and_request_indices_known_answer() -> None:
    c = GOLDEN["visibility_packing"]
    md = lv.PagedAttentionMetadata(
        block_tables=tuple(tuple(t) for t in c["block_tables"]),
        num_computed_tokens=tuple(c["num_computed_tokens"]),
        query_layouts=tuple(lv.QueryLayout(tuple(p)) for p in c["layouts"]),
    )
    vis, starts = md.visibility_tensor(device=CPU)
    assert vis.tolist() == c["visibility"]
    assert starts.tolist() == c["visibility_start"]
    assert md.query_start_loc == tuple(c["query_start_loc"])
    assert md.request_indices_tensor(device=CPU).tolist() == c["request_indices"]
    assert not md.has_only_linear_queries


def test_layout_known_answers() -> None:
    c = GOLDEN["query_layout"]
    layout = lv.QueryLayout(tuple(c["parents"]))
    assert list(lv.semantic_positions(layout, prefix_length=c["prefix_length"])) == c["positions"]
    assert [list(r) for r in lv.query_visibility(layout)] == c["visibility"]
    d = c["append_draft"]
    draft = lv.DraftTree((7, 9, 8), tuple(d["draft_parents"]))
    assert list(lv.append_draft_layout(d["num_inputs"], draft).parent_indices) == d["expected"]
    with pytest.raises(ValueError, match="precede"):
        lv.DraftTree((4, 5), (-1, 1))
    with pytest.raises(ValueError, match="siblings"):
        lv.DraftTree((4, 4), (-1, -1))


def test_visible_logical_positions_known_answer() -> None:
    c = GOLDEN["visible_positions"]
    md = lv.PagedAttentionMetadata(
        block_tables=((2, 0),), num_computed_tokens=(c["num_computed_tokens"],),
        query_layouts=(lv.QueryLayout(tuple(c["parents"])),),
    )
    assert [list(p) for p in md.visible_logical_positions(0)] == c["expected"]


def _random_metadata(rng, *, batch, bs, tree=False):
    computed = [int(x) for x in rng.integers(0, 60, size=batch)]
    layouts = []
    for _ in range(batch):
        q = int(rng.integers(1, 40))
        if tree:
            parents = tuple([-1] + [int(rng.integers(0, i)) for i in range(1, q)])
        else:
            parents = tuple(range(-1, q - 1))
        layouts.append(lv.QueryLayout(parents))
    reserved = [len(l) + int(rng.integers(0, 3)) for l in layouts]
    need = [(c + r + bs - 1) // bs for c, r in zip(computed, reserved)]
    perm = [int(x) for x in rng.permutation(sum(need) + 5)]
    tables, off = [], 0
    for n in need:
        tables.append(tuple(perm[off : off + n]))
        off += n
    return lv.PagedAttentionMetadata(
        block_tables=tuple(tables), num_computed_tokens=tuple(computed), query_layouts=tuple(layouts),
        num_reserved_query_tokens=tuple(reserved),
    )


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("bs", (1, 3, 16))
def test_plan_slots_match_oracle_slot_mapping(seed, bs) -> None:
    rng = np.random.default_rng(seed)
    md = _random_metadata(rng, batch=7, bs=bs, tree=seed % 2 == 1)
    plan = StepPlan(md, block_size=bs, device=CPU)
    expect = O.slot_mapping(md.block_tables, md.num_computed_tokens, md.query_lengths,
                            md.num_reserved_query_tokens, bs)
    assert plan.slots.tolist() == expect.tolist()
    assert plan.slots.tolist() == md.slot_mapping(block_size=bs, device=CPU).tolist()


@pytest.mark.parametrize("seed", range(3))
def test_plan_visibility_bits_match_oracle(seed) -> None:
    rng = np.random.default_rng(100 + seed)
    md = _random_metadata(rng, batch=5, bs=4, tree=True)
    plan = StepPlan(md, block_size=4, device=CPU)
    meta = plan.req_meta.view(-1, native.REQ_FIELDS).numpy()
    words = plan.vis.numpy().view(np.uint32)
    for r, layout in enumerate(md.query_layouts):
        vis = O.query_visibility(layout.parent_indices)
        if O.is_linear(layout.parent_indices):
            assert meta[r, 5] == -1
            continue
        off, w = meta[r, 5], meta[r, 6]
        q = len(layout)
        for i in range(q):
            for j in range(q):
                bit = (int(words[off + i * w + j // 32]) >> (j % 32)) & 1
                assert bit == int(vis[i, j])


def test_plan_request_table_matches_metadata() -> None:
    rng = np.random.default_rng(9)
    md = _random_metadata(rng, batch=9, bs=16)
    plan = StepPlan(md, block_size=16, device=CPU)
    meta = plan.req_meta.view(-1, native.REQ_FIELDS).numpy()
    assert meta[:, 2].tolist() == list(md.num_computed_tokens)
    assert meta[:, 3].tolist() == list(md.query_lengths)
    assert meta[:, 4].tolist() == list(md.query_start_loc[:-1])
    flat = plan.tables.numpy()
    for r, table in enumerate(md.block_tables):
        assert flat[meta[r, 0] : meta[r, 0] + meta[r, 1]].tolist() == list(table)


@pytest.mark.parametrize("unit,ctw", ((16, 1), (32, 1), (64, 1), (16, 4), (64, 4)))
@pytest.mark.parametrize("resident", (7, 64, 2048))
@pytest.mark.parametrize("bs", (1, 16))
@pytest.mark.parametrize("group", (1, 7))
def test_stream_k_pieces_cover_every_segment_once(resident, bs, group, unit, ctw) -> None:
    rng = np.random.default_rng(resident + bs + group + unit + ctw)
    md = _random_metadata(rng, batch=11, bs=bs)
    plan = StepPlan(md, block_size=bs, device=CPU)
    work = plan.work(group, 4, resident, 0, unit, ctw)
    assert work.col_tiles == ctw
    pieces = work.pieces.numpy()
    first = work.wave_first.numpy()
    waves = work.waves_per_head
    assert first[0] == 0 and first[-1] == len(pieces) and np.all(np.diff(first) >= 1)
    u = unit
    cap = (254 * bs) // u  # units whose block-table slice fits the kernel's LDS copy
    assert work.units_per_wave <= max(cap, 1)
    seqs = np.asarray(md.num_computed_tokens) + np.asarray(md.query_lengths)
    ngroups = -(-(-(-(np.asarray(md.query_lengths) * group) // 16)) // ctw)
    total_tiles = int((-(-seqs // u) * ngroups).sum())
    assert waves <= max(resident // 4, 1, -(-total_tiles // cap))
    assert work.units_per_wave == -(-total_tiles // waves)
    share_sizes = []
    covered = {}
    for w in range(waves):
        tiles = 0
        for rec in pieces[first[w] : first[w + 1]]:
            req, ctile, tb, te, slot = rec[:5]
            assert 0 <= tb < te <= seqs[req] and tb % u == 0
            assert rec[6] == md.num_computed_tokens[req] and rec[7] == md.query_lengths[req]
            assert rec[8] == md.query_start_loc[req]
            n_tab = (te - 1) // bs - tb // bs + 1
            assert n_tab <= 254, "piece exceeds the kernel's LDS table slice"
            covered.setdefault((req, ctile), []).append((tb, te, slot))
            table = md.block_tables[req]
            for j in range(5):  # first-tile block ids carried by the piece
                lb = tb // bs + j
                assert rec[11 + j] == (table[lb] if lb < len(table) else 0)
            tiles += -(-(te - tb) // u)
        assert tiles <= work.units_per_wave
        share_sizes.append(tiles)
        # Only a share's first and last pieces can be partial.
        wave_slots = pieces[first[w] : first[w + 1], 4]
        assert all(sl < 0 for sl in wave_slots[1:-1])
    assert max(share_sizes) - min(share_sizes) <= 1 and sum(share_sizes) == total_tiles
    job_rows = work.jobs.numpy() if work.num_jobs else []
    jobs = {(int(j[0]), int(j[1])): (int(j[2]), int(j[3])) for j in job_rows}
    for j in job_rows:  # the merge kernel reads q_start and q_len from the job
        assert j[4] == md.query_start_loc[j[0]] and j[5] == md.query_lengths[j[0]]
        assert j[3] <= 48  # pieces per segment (the planner's cap)
    slots_seen = []
    for r, q in enumerate(md.query_lengths):
        for ct in range(ngroups[r]):
            spans = sorted(covered[(r, ct)])
            assert spans[0][0] == 0 and spans[-1][1] == seqs[r]
            assert all(a[1] == b[0] for a, b in zip(spans, spans[1:]))
            if len(spans) == 1:
                assert spans[0][2] == -1 and (r, ct) not in jobs
            else:
                s0, n = jobs[(r, ct)]
                assert [sp[2] for sp in spans] == list(range(s0, s0 + n)) and n == len(spans)
                slots_seen += list(range(s0, s0 + n))
    assert sorted(slots_seen) == list(range(work.num_partial_slots))


@pytest.mark.parametrize("computed, waves", ((1024, 33), (2048, 33), (4096, 43), (300, 10)))
def test_stream_k_cuts_no_segment_into_more_than_48_pieces(computed, waves) -> None:
    """One sequence on stream-K shares: one tile per share while that cuts it
    into at most 48 pieces (the merge reads 16 partials per round trip),
    longer shares past that (65 tiles: 33 shares of two; 129: 43 of three)."""

    md = lv.PagedAttentionMetadata(block_tables=(tuple(range(-(-(computed + 1) // 16))),),
                                   num_computed_tokens=(computed,),
                                   query_layouts=(lv.linear_query_layout(1),))
    plan = StepPlan(md, block_size=16, device=CPU)
    work = plan.work(7, 4, 1024, 0, 32, 1)
    assert work.waves_per_head == waves and work.group_waves == 1
    assert work.num_jobs == 1 and int(work.jobs.numpy()[0][3]) == waves <= 48


@pytest.mark.parametrize("gw", (4, 8))
@pytest.mark.parametrize("bs", (1, 16))
@pytest.mark.parametrize("seed", range(6))
def test_workgroup_split_gives_each_segment_one_workgroup(seed, bs, gw) -> None:
    """A latency-bound decode step (short segments that fit the resident
    workgroups) runs one segment per workgroup of ``gw`` waves, one record
    per wave: workgroup b's records are the segment's near-equal contiguous
    parts from wave gw*b on, then idle records (request -1); no merge jobs or
    partial slots; a single-piece segment is written by its piece (slot -1),
    the others name their wave."""

    rng = np.random.default_rng(900 + seed)
    batch = int(rng.integers(1, 20))
    computed = tuple(int(c) for c in rng.integers(0, 400, size=batch))
    need = [-(-(c + 1) // bs) for c in computed]
    perm = [int(x) for x in rng.permutation(sum(need) + 3)]
    tables, off = [], 0
    for n in need:
        tables.append(tuple(perm[off : off + n]))
        off += n
    md = lv.PagedAttentionMetadata(block_tables=tuple(tables), num_computed_tokens=computed,
                                   query_layouts=tuple(lv.linear_query_layout(1) for _ in range(batch)))
    plan = StepPlan(md, block_size=bs, device=CPU)
    unit = 32
    work = plan.work(7, 4, 1024, 0, unit, 1, split_groups=256, split_waves=gw)
    seqs = np.asarray(computed) + 1
    tiles = -(-seqs // unit)
    stream_k = plan.work(7, 4, 1024, 0, unit, 1)
    split = -(-int(tiles.max()) // gw)
    cap = (254 * bs) // unit
    longest = int(tiles.max())
    use = batch * 4 <= 256 and split <= min(cap, 2) and split <= stream_k.units_per_wave + (
        3 if stream_k.num_jobs else 0)
    if split == 2 and 2 * longest > 3 * gw and batch * 4 < 128:
        use = False
    if not use:
        assert work.group_waves == 1 and work.waves_per_head == stream_k.waves_per_head
        return
    assert work.group_waves == gw and work.waves_per_head == gw * batch
    assert work.num_jobs == 0 and work.num_partial_slots == 0 and work.units_per_wave == split
    pieces = work.pieces.numpy()
    first = work.wave_first.numpy()
    assert pieces.shape[0] == gw * batch and first.tolist() == list(range(gw * batch + 1))
    for r in range(batch):
        block = pieces[gw * r : gw * (r + 1)]
        n = min(gw, int(tiles[r]))
        assert [int(x[0]) for x in block] == [r] * n + [-1] * (gw - n)  # the first n waves, then idle
        recs = block[:n]
        assert recs[0][2] == 0 and recs[-1][3] == seqs[r]
        assert all(a[3] == b[2] for a, b in zip(recs, recs[1:]))
        assert [int(x[4]) for x in recs] == ([-1] if n == 1 else list(range(n)))
        assert all(int(x[4]) == -1 for x in block[n:])
        for x in recs:
            assert x[2] % unit == 0
            assert -(-(int(x[3]) - int(x[2])) // unit) in (tiles[r] // n, -(-int(tiles[r]) // n))
            for j in range(5):
                lb = x[2] // bs + j
                assert x[11 + j] == (tables[r][lb] if lb < len(tables[r]) else 0)


def test_workgroup_split_is_not_used_where_stream_k_is_faster() -> None:
    # C2-like contexts U[512, 4096]: stream-K shares are far shorter than a
    # quarter of the longest segment.  (Equal long contexts split evenly in
    # workgroups, which then need no merge.)
    rng = np.random.default_rng(1)
    computed = tuple(int(c) for c in rng.integers(512, 4097, size=64))
    need = [-(-(c + 1) // 16) for c in computed]
    tables = tuple(tuple(range(sum(need[:r]), sum(need[: r + 1]))) for r in range(64))
    md = lv.PagedAttentionMetadata(block_tables=tables, num_computed_tokens=computed,
                                   query_layouts=tuple(lv.linear_query_layout(1) for _ in range(64)))
    plan = StepPlan(md, block_size=16, device=CPU)
    for gw in (4, 8):
        assert plan.work(7, 4, 1024, 0, 32, 1, split_groups=256, split_waves=gw).group_waves == 1
    # Equal contexts: more than two tiles per wave stays on stream-K; two
    # take the split when the pieces average at most 1.5 tiles or the step
    # has 128 segments or more; one always does.
    for batch, computed, gw in ((64, 4000, 1), (64, 1000, 1), (8, 600, 1), (8, 500, 1), (32, 500, 8),
                                (8, 380, 8), (8, 250, 8), (1, 0, 8)):
        plan = StepPlan(_uniform_metadata(batch=batch, computed=computed, q=1), block_size=16, device=CPU)
        got = plan.work(7, 4, 1024, 0, 32, 1, split_groups=256, split_waves=8).group_waves
        assert got == gw, (batch, computed, got)
    plan = StepPlan(_uniform_metadata(batch=70, computed=100, q=1), block_size=16, device=CPU)
    assert plan.work(7, 4, 1024, 0, 32, 1, split_groups=256).group_waves == 1  # 280 workgroups > 256
    assert plan.work(7, 4, 1024, 0, 32, 1, split_groups=512).group_waves == 8
    # Four column tiles per wave never split in workgroups.
    plan = StepPlan(_uniform_metadata(batch=4, computed=100, q=8), block_size=16, device=CPU)
    assert plan.work(7, 4, 1024, 0, 16, 4, split_groups=256).group_waves == 1


def _uniform_metadata(*, batch, computed, q, bs=16):
    layouts = tuple(lv.QueryLayout(tuple(range(-1, q - 1))) for _ in range(batch))
    need = -(-(computed + q) // bs)
    tables = tuple(tuple(range(r * need, (r + 1) * need)) for r in range(batch))
    return lv.PagedAttentionMetadata(
        block_tables=tables, num_computed_tokens=(computed,) * batch, query_layouts=layouts,
        num_reserved_query_tokens=(q,) * batch,
    )


def test_col_tiles_choice_follows_the_reread_cost() -> None:
    from light_vllm_amd.plan import COL_TILES4_COST
    # One column tile per request (decode at group 7): nothing to share.
    plan = StepPlan(_uniform_metadata(batch=4, computed=500, q=1), block_size=16, device=CPU)
    assert plan.choose_col_tiles(7, 0, 4) == 1
    # Eight queries x group 7 = 4 column tiles: one wave reads K/V once, not 4 times.
    plan = StepPlan(_uniform_metadata(batch=4, computed=500, q=8), block_size=16, device=CPU)
    assert plan.choose_col_tiles(7, 0, 4) == (4 if COL_TILES4_COST < 4 else 1)
    assert plan.choose_col_tiles(7, 0, 1) == 1  # the kernel is not built for this shape
    # Three queries x group 7 = 2 column tiles: four tiles pay off only below cost 2.
    plan = StepPlan(_uniform_metadata(batch=4, computed=500, q=3), block_size=16, device=CPU)
    assert plan.choose_col_tiles(7, 0, 4) == (4 if COL_TILES4_COST < 2 else 1)


@pytest.mark.parametrize("group,columns", ((7, 256), (1, 256), (4, 128)))
@pytest.mark.parametrize("resident", (0, 64, 4096))
@pytest.mark.parametrize("key_tokens", (32, 64))
def test_prefill_pieces_cover_every_wide_request_once(group, columns, resident, key_tokens) -> None:
    """Every (column, key) pair of a wide request is in exactly one prefill
    piece; split units' pieces own consecutive partial slots that one merge
    job names; pieces are heaviest first."""

    rng = np.random.default_rng(12 + group + resident)
    md = _random_metadata(rng, batch=6, bs=16)
    plan = StepPlan(md, block_size=16, device=CPU)
    work = plan.work(group, 4, 2048, columns, 64, 1, key_tokens, resident)
    computed = np.asarray(md.num_computed_tokens)
    units = work.prefill_units.numpy() if work.num_prefill_units else np.zeros((0, 8), np.int32)
    spans: dict[tuple[int, int], list] = {}
    work_prev = None
    table_off = np.concatenate(([0], np.cumsum([len(t) for t in md.block_tables])))
    for req, c0, n, kb, ke, slot, toff, qs, comp, ql, voff, vwords, *first in units:
        assert 0 < n <= columns and c0 % columns == 0
        assert (toff, qs, comp, ql, vwords) == (table_off[req], md.query_start_loc[req], computed[req],
                                                md.query_lengths[req], 0) and voff == -1
        lb0, table = kb // 16, md.block_tables[req]
        assert first == [table[lb0 + b] if lb0 + b < len(table) else 0 for b in range(4)]
        kneed = computed[req] + (c0 + n - 1) // group + 1
        end = ke if ke else kneed
        assert kb % key_tokens == 0 and kb < end <= kneed and (ke == 0 or ke % key_tokens == 0)
        spans.setdefault((int(req), int(c0)), []).append((int(kb), int(end), int(slot), int(n)))
        w = -(-(end - kb) // key_tokens) * n
        assert work_prev is None or w <= work_prev  # heaviest first
        work_prev = w
    jobs = {(int(j[0]), int(j[1])): j for j in (work.prefill_jobs.numpy() if work.num_prefill_jobs else [])}
    slots = []
    for (req, c0), sp in spans.items():
        sp.sort()
        kneed = computed[req] + (c0 + sp[0][3] - 1) // group + 1
        assert sp[0][0] == 0 and sp[-1][1] == kneed
        assert all(a[1] == b[0] for a, b in zip(sp, sp[1:]))
        if len(sp) == 1:
            assert sp[0][2] == -1 and (req, c0 // columns) not in jobs
        else:
            j = jobs[(req, c0 // columns)]
            assert [x[2] for x in sp] == list(range(j[2], j[2] + j[3])) and j[3] == len(sp)
            assert j[4] == md.query_start_loc[req] and j[5] == md.query_lengths[req]
            assert all(-(-(x[1] - x[0]) // key_tokens) >= 4 or x is sp[-1] for x in sp)
            slots += [x[2] for x in sp]
    assert sorted(slots) == list(range(work.num_prefill_partial_slots))
    if resident == 0:
        assert work.num_prefill_partial_slots == 0  # no split without a resident count
    decode_reqs = set()
    if work.waves_per_head:
        decode_reqs = {int(r) for r in work.pieces.numpy()[:, 0]}
    for r, q in enumerate(md.query_lengths):
        if q * group > 16:
            cols = sorted(c for (rr, c0), sp in spans.items() if rr == r for c in range(c0, c0 + sp[0][3]))
            assert cols == list(range(q * group)) and r not in decode_reqs
        else:
            assert all(rr != r for rr, _ in spans) and r in decode_reqs
    # Without the prefill kernel every request is a decode row.
    assert plan.work(group, 4, 2048, 0).num_prefill_units == 0


def _prefix_metadata(rng, groups, *, bs, decode_between=False):
    """Requests in groups sharing a readonly prefix of ``shared`` blocks each
    (one (n, shared, q_range) per group), draft trees of q queries; with
    ``decode_between`` a one-query request follows every group."""

    tables, computed, layouts, readonly = [], [], [], []
    nxt = 0
    for n, shared, (qlo, qhi) in groups:
        prefix = list(range(nxt, nxt + shared))
        nxt += shared
        for _ in range(n):
            c = shared * bs + int(rng.integers(0, 200))
            q = int(rng.integers(qlo, qhi + 1))
            parents = tuple([-1] + [int(rng.integers(0, i)) for i in range(1, q)])
            need = -(-(c + q) // bs)
            tables.append(tuple(prefix + list(range(nxt, nxt + need - shared))))
            nxt += need - shared
            computed.append(c)
            layouts.append(lv.QueryLayout(parents))
            readonly.append(shared)
        if decode_between:
            c = int(rng.integers(1, 300))
            need = -(-(c + 1) // bs)
            tables.append(tuple(range(nxt, nxt + need)))
            nxt += need
            computed.append(c)
            layouts.append(lv.QueryLayout((-1,)))
            readonly.append(0)
    md = lv.PagedAttentionMetadata(block_tables=tuple(tables), num_computed_tokens=tuple(computed),
                                   query_layouts=tuple(layouts), num_readonly_prefix_blocks=tuple(readonly))
    return md, nxt


def _check_prefill_coverage(md, work, *, group, columns, key_tokens, bs):
    """Every (column, key) pair of every wide request is covered exactly once:
    by its own units' pieces, or, below a span's prefix, by the pieces of the
    span unit holding the column; every merge job names exactly those pieces'
    partial slots; spans only cover blocks all their members list at the same
    logical index, below every member's computed count.  Returns the spans
    found (first token -> prefix tokens)."""

    computed = np.asarray(md.num_computed_tokens)
    q_start = np.asarray(md.query_start_loc)
    flat = [b for t in md.block_tables for b in t]
    units = work.prefill_units.numpy() if work.num_prefill_units else np.zeros((0, 16), np.int32)
    pads = units[:, 2] == 0  # padding records of the per-XCD order
    assert (units[pads, 0] == PAD_RECORD).all() and (units[pads, 5] == -1).all()
    units = units[~pads]
    jobs = work.prefill_jobs.numpy() if work.num_prefill_jobs else np.zeros((0, 8), np.int32)
    own: dict[tuple[int, int], list] = {}
    span_units: dict[int, list] = {}  # first token -> [(col0, n, kb, ke, slot)]
    starts = np.concatenate(([0], np.cumsum([len(t) for t in md.block_tables])))
    for req, c0, n, kb, ke, slot, table_off, t0, comp, ql, voff, vwords, *first in units.tolist():
        assert 0 < n <= columns and c0 % columns == 0 and kb % key_tokens == 0
        lb0, lb1 = kb // bs, (kb + key_tokens - 1) // bs
        if lb1 - lb0 >= 4:  # else the first tile's block ids ride in the record
            assert first[0] == -1
        if req < 0:
            assert ke > kb and ke % key_tokens == 0 and slot >= 0
            assert (comp, ql, voff, vwords) == (ke, 0, -1, 0)
            if lb1 - lb0 < 4:  # the blocks the piece's first tile reads
                used = range(lb0, min(lb1, (ke - 1) // bs) + 1)
                assert [first[b - lb0] for b in used] == [flat[table_off + b] for b in used]
            span_units.setdefault(t0, []).append((c0, n, kb, ke, slot, table_off))
        else:
            assert (table_off, t0, comp, ql) == (starts[req], q_start[req], computed[req], md.query_lengths[req])
            if lb1 - lb0 < 4:
                table = md.block_tables[req]
                assert first == [table[lb0 + b] if lb0 + b < len(table) else 0 for b in range(4)]
            kneed = computed[req] + (c0 + n - 1) // group + 1
            own.setdefault((req, c0), []).append((kb, ke if ke else kneed, slot, n, kneed))
    used_slots = [u[5] for u in units.tolist() if u[5] >= 0]
    assert sorted(used_slots) == list(range(work.num_prefill_partial_slots))
    job_of = {(int(j[0]), int(j[1])): j for j in jobs}
    spans = {}
    for (req, c0), pieces in own.items():
        pieces.sort()
        kneed = pieces[0][4]
        assert pieces[-1][1] == kneed and all(a[1] == b[0] for a, b in zip(pieces, pieces[1:]))
        job = job_of.get((req, c0 // columns))
        start = pieces[0][0]
        if start == 0 and len(pieces) == 1 and pieces[0][2] == -1:
            assert job is None
            continue
        assert job is not None and list(job[2:4]) == [pieces[0][2], len(pieces)]
        assert [p[2] for p in pieces] == list(range(job[2], job[2] + job[3]))
        assert job[4] == q_start[req] and job[5] == md.query_lengths[req]
        if start == 0:
            assert job[6] == 0
            continue
        # Keys [0, start) come from the request's span.
        k = int(job[7]) >> 24
        v0 = int(job[7]) & 0xFFFFFF
        t0 = int(q_start[req]) - v0 // group
        assert v0 % group == 0 and t0 in span_units and k >= 1
        su = sorted(span_units[t0])
        assert start == max(x[3] for x in su) and start % key_tokens == 0 and start <= computed[req]
        spans[t0] = start
        assert len({x[5] for x in su}) == 1
        table_off, blocks = su[0][5], -(-start // bs)
        assert md.block_tables[req][:blocks] == tuple(flat[table_off : table_off + blocks])
        base = int(job[6]) - 1
        for c in range(c0, c0 + pieces[0][3]):
            v = v0 + c
            mine = sorted((x[2], x[3], x[4]) for x in su if x[0] <= v < x[0] + x[1])
            assert mine[0][0] == 0 and mine[-1][1] == start and all(a[1] == b[0] for a, b in zip(mine, mine[1:]))
            assert [x[2] for x in mine] == list(range(base + (v // columns) * k, base + (v // columns) * k + k))
    for r, q in enumerate(md.query_lengths):
        if q * group > 16:
            cols = sorted(c for (rr, c0), p in own.items() if rr == r for c in range(c0, c0 + p[0][3]))
            assert cols == list(range(q * group))
    return spans


@pytest.mark.parametrize("seed", range(8))
@pytest.mark.parametrize("bs", (1, 12, 16))
def test_shared_prefix_spans_cover_every_key_once(seed, bs) -> None:
    """Shared-prefix spans (C5's shape and mixtures): coverage, merge slots,
    and the span's blocks, against the metadata itself."""

    rng = np.random.default_rng(700 + seed)
    groups = [(int(rng.integers(1, 9)), int(rng.integers(0, 700 // bs + 2)), (3, 12)) for _ in range(3)]
    md, nb = _prefix_metadata(rng, groups, bs=bs, decode_between=seed % 2 == 1)
    plan = StepPlan(md, block_size=bs, device=CPU, num_blocks=nb)
    for resident in (0, 256):
        work = plan.work(6, 2, 2048, 128, 64, 1, 64, resident, 8, shared_prefix=True)
        spans = _check_prefill_coverage(md, work, group=6, columns=128, key_tokens=64, bs=bs)
        ref = plan.work(6, 2, 2048, 128, 64, 1, 64, resident, 8, shared_prefix=False)
        assert _check_prefill_coverage(md, ref, group=6, columns=128, key_tokens=64, bs=bs) == {}
        # A group over a prefix of two or more key tiles whose trees pack into
        # fewer 128-column units than they take one by one forms a span.
        r = 0
        for n, shared, _ in groups:
            cols = sum(md.query_lengths[i] * 6 for i in range(r, r + n))
            if n >= 2 and shared * bs >= 2 * 64 and -(-cols // 128) < n:
                assert spans.get(md.query_start_loc[r]) == shared * bs // 64 * 64
            r += n + (seed % 2)


def test_shared_prefix_span_shapes() -> None:
    """C5's step: 32 trees of 9 queries at group 6 over a 2,032-token readonly
    prefix form one span of 1,728 columns: 14 span units over the prefix's
    1,984 tile-aligned tokens, each member's own units from there.  Requests
    of a full unit each, or prefixes under two key tiles, form none."""

    rng = np.random.default_rng(5)
    md, nb = _prefix_metadata(rng, [(32, 127, (9, 9))], bs=16)
    plan = StepPlan(md, block_size=16, device=CPU, num_blocks=nb)
    work = plan.work(6, 2, 2048, 128, 64, 1, 64, 256, 8, shared_prefix=True)
    spans = _check_prefill_coverage(md, work, group=6, columns=128, key_tokens=64, bs=16)
    assert spans == {0: 1984}
    units = work.prefill_units.numpy()
    assert len({tuple(u[1:3]) for u in units if u[0] < 0}) == 14
    md, nb = _prefix_metadata(rng, [(4, 127, (16, 16))], bs=16)  # 16 x 8 = 128 columns each
    work = StepPlan(md, block_size=16, device=CPU, num_blocks=nb).work(8, 1, 2048, 128, 64, 1, 64, 256, 8,
                                                                       shared_prefix=True)
    assert not (work.prefill_units.numpy()[:, 0] < 0).any()
    md, nb = _prefix_metadata(rng, [(8, 7, (9, 9))], bs=16)  # 112 shared tokens: under two tiles
    work = StepPlan(md, block_size=16, device=CPU, num_blocks=nb).work(6, 2, 2048, 128, 64, 1, 64, 256, 8,
                                                                       shared_prefix=True)
    assert not (work.prefill_units.numpy()[:, 0] < 0).any()


PAD_RECORD = 2**31 - 1


def _record_work(u, group, key_tokens):
    """Key tiles x columns of one prefill record (the planner's balance measure)."""

    kneed = u[8] + (u[1] + u[2] - 1) // group + 1
    kmax = u[4] if 0 < u[4] < kneed else kneed
    return (-(-kmax // key_tokens) - u[3] // key_tokens) * u[2]


@pytest.mark.parametrize("hkv", (1, 2, 3, 4, 8, 28))
@pytest.mark.parametrize("seed", range(6))
def test_prefill_grid_is_ordered_per_xcd(hkv, seed) -> None:
    """With 8 XCDs the grid's workgroup b = (position b / H, kv head b % H)
    runs on XCD b % 8, so positions congruent modulo P = 8 / gcd(H, 8) share
    an XCD per kv head.  The ordered lists hold the unordered ones' records
    plus padding, P bins interleaved, each bin heaviest first, and the bins
    balanced to within one record (or 1/32 of a bin)."""

    rng = np.random.default_rng(700 + seed)
    group, key_tokens = 7 if hkv <= 4 else 1, 64
    n = int(rng.integers(2, 10))
    computed = [int(c) for c in rng.integers(0, 3000, size=n)]
    q_lens = [int(q) for q in rng.integers(40, 600, size=n)]
    need = [(c + q + 15) // 16 for c, q in zip(computed, q_lens)]
    perm = [int(x) for x in rng.permutation(sum(need) + 5)]
    tables, off = [], 0
    for k in need:
        tables.append(tuple(perm[off: off + k]))
        off += k
    md = lv.PagedAttentionMetadata(block_tables=tuple(tables), num_computed_tokens=tuple(computed),
                                   query_layouts=tuple(lv.linear_query_layout(q) for q in q_lens))
    plan = StepPlan(md, block_size=16, device=CPU)
    args = (group, hkv, 2048, 128, 64, 1, key_tokens, 0)
    flat = plan.work(*args, xcds=0).prefill_units.numpy()
    work = plan.work(*args, xcds=8, prefill_order=1)
    _check_prefill_coverage(md, work, group=group, columns=128, key_tokens=key_tokens, bs=16)
    units = work.prefill_units.numpy()
    bins = 8 // math.gcd(hkv, 8)
    assert len(units) % bins == 0
    real = units[units[:, 2] > 0]
    assert sorted(map(tuple, real.tolist())) == sorted(map(tuple, flat.tolist()))
    load = [0] * bins
    works = [_record_work(u, group, key_tokens) for u in units.tolist()]
    for b in range(bins):
        seq = [w for k, w in enumerate(works) if k % bins == b and units[k, 2] > 0]
        assert seq == sorted(seq, reverse=True)  # heaviest first
        load[b] = sum(seq)
    gap = max(load) - min(load)
    assert gap * 32 * bins <= sum(load) or gap <= max(works)
    if bins == 1:
        assert len(real) == len(units)


def _makespan(units, bins, slots, group, key_tokens):
    """Latest finish over the bins when each bin's records start in order,
    each on the first of ``slots`` slots to free (padding: nothing)."""

    import heapq

    worst = 0
    for b in range(bins):
        heap = [0] * slots
        for u in units.tolist()[b::bins]:
            if u[2] > 0:
                heapq.heappush(heap, heapq.heappop(heap) + _record_work(u, group, key_tokens))
        worst = max(worst, max(heap))
    return worst


@pytest.mark.parametrize("seed", range(8))
def test_auto_prefill_order_keeps_the_faster_packing(seed) -> None:
    """``prefill_order`` 0 (auto) returns the grouped order when its packing
    of the resident slots is at most 1/64 slower than the plain heaviest-first
    order's, else the plain order."""

    rng = np.random.default_rng(900 + seed)
    n = int(rng.integers(2, 12))
    computed = [int(c) for c in rng.integers(0, 4000, size=n)]
    q_lens = [int(q) for q in rng.integers(64, 700, size=n)]
    need = [(c + q + 15) // 16 for c, q in zip(computed, q_lens)]
    perm = [int(x) for x in rng.permutation(sum(need) + 5)]
    tables, off = [], 0
    for k in need:
        tables.append(tuple(perm[off: off + k]))
        off += k
    md = lv.PagedAttentionMetadata(block_tables=tuple(tables), num_computed_tokens=tuple(computed),
                                   query_layouts=tuple(lv.linear_query_layout(q) for q in q_lens))
    plan = StepPlan(md, block_size=16, device=CPU)
    hkv, slots = 4, 128  # 512 resident workgroups over 4 kv heads
    args = (7, hkv, 2048, 128, 64, 1, 64, slots * hkv)
    auto = plan.work(*args, xcds=8, prefill_order=0).prefill_units.numpy()
    grouped = plan.work(*args, xcds=8, prefill_order=1).prefill_units.numpy()
    plain = plan.work(*args, xcds=8, prefill_order=2).prefill_units.numpy()
    assert plain.tolist() == plan.work(*args, xcds=0).prefill_units.numpy().tolist()
    mg, mp = (_makespan(u, 2, slots // 2, 7, 64) for u in (grouped, plain))
    assert auto.tolist() == (grouped if mg * 64 <= mp * 65 else plain).tolist()


def test_prefill_split_fills_the_resident_workgroups() -> None:
    # C5-like: tree verification of 9 queries at group 6 = 54 columns, one
    # unit per request; 4 requests x 32 key tiles over 16 slots per kv head.
    plan = StepPlan(_uniform_metadata(batch=4, computed=2000, q=9), block_size=16, device=CPU)
    work = plan.work(6, 2, 2048, 128, 64, 1, 64, 32)
    assert work.waves_per_head == 0 and work.num_prefill_units == 16
    assert work.num_prefill_jobs == 4 and work.num_prefill_partial_slots == 16
    units = work.prefill_units.numpy()
    assert sorted(units[:, 3].tolist()) == sorted([0, 512, 1024, 1536] * 4)
    assert sorted(units[:, 4].tolist()) == sorted([512, 1024, 1536, 0] * 4)


def test_merge_grids_cover_only_the_columns_jobs_use() -> None:
    # Tree verification at group 6: 9 x 6 = 54 of a prefill slot's 128 columns.
    plan = StepPlan(_uniform_metadata(batch=4, computed=2000, q=9), block_size=16, device=CPU)
    work = plan.work(6, 2, 2048, 128, 64, 1, 64, 32)
    assert work.num_prefill_jobs == 4 and work.prefill_merge_columns == 54
    # Decode at group 7: 7 of a decode slot's 16 columns.
    plan = StepPlan(_uniform_metadata(batch=8, computed=3000, q=1), block_size=16, device=CPU)
    work = plan.work(7, 4, 1024, 128, 64, 1, 64, 32)
    assert work.num_jobs > 0 and work.merge_columns == 7
    # 40 queries at group 7 = 280 columns: units of 128, 128 and 24.
    plan = StepPlan(_uniform_metadata(batch=1, computed=3000, q=40), block_size=16, device=CPU)
    work = plan.work(7, 4, 1024, 128, 64, 1, 64, 256)
    assert work.num_prefill_jobs == 3 and work.prefill_merge_columns == 128


def test_library_loads_and_exports_every_header_function() -> None:
    lib = native.load()
    declared = native.header_functions()
    assert declared, "no functions parsed from the header"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
        assert name in native.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.lvamd_abi_version() == native.ABI_VERSION
    assert lib.lvamd_status_string(-3).decode() == "workspace missing or too small"
    assert lib.lvamd_kv_compact_inline_pairs() == 32
    assert lib.lvamd_kv_compact_workspace_size(32, 28, 1024) == 0
    assert lib.lvamd_kv_compact_workspace_size(33, 28, 1024) == 33 * 28 * 2 * 1024
    # The small compact takes at most the inline pair count (refused before any HIP call).
    assert lib.lvamd_kv_compact_small(None, None, 28, 1024, None, None, 33, None) == -1
    # The one-pass compact checks its arguments before any HIP call.
    assert lib.lvamd_kv_compact_ordered(None, None, 28, 1024, None, None, None, 0, None) == 0
    assert lib.lvamd_kv_compact_ordered(None, None, 28, 1024, None, None, None, 2, None) == -1
    assert lib.lvamd_kv_compact_ordered(None, None, 0, 1024, None, None, None, 2, None) == -1
    assert lib.lvamd_kv_block_copy_small_pairs() == 32
    assert lib.lvamd_kv_block_copy_small(None, None, 28, 8192, None, None, 33, None) == -1
    # The allocation-free compact refuses, before any HIP call, a call whose
    # staged rows exceed its static scratch (16 MiB): 16 MiB / (28 * 2 * 1024) = 292 pairs.
    assert lib.lvamd_kv_compact_static(None, None, 28, 1024, None, None, 293, None) == -5
    assert lib.lvamd_kv_compact_static(None, None, 28, 1 << 40, None, None, 33, None) == -5
    assert "static scratch" in lib.lvamd_status_string(-5).decode()
    # Argument checks run before any HIP call, so they are safe without a GPU.
    assert lib.lvamd_kv_append(None, 0, 0, None, 0, 0, None, None, None, 1, 2, 64, 2, None) == -1
    no_append = (None, 0, 0, None, 0, 0)
    assert lib.lvamd_paged_decode(None, 0, 0, *no_append, None, None, None, 0, 0, None, None, 1, None, None,
                                  None, None, 0, 4, 7, 72, 1, 1, 16, ctypes.c_float(0.1), 2, None) == -2
    # Head sizes: multiples of 16 from 32 to 256 pass the shape check (and
    # stop at the null pointers), others are not built.
    for d, want in ((48, -1), (112, -1), (240, -1), (16, -2), (40, -2), (264, -2), (272, -2)):
        for dtype in (0, 1, 2):
            assert lib.lvamd_paged_decode(None, 0, 0, *no_append, None, None, None, 0, 0, None, None, 1, None, None,
                                          None, None, 0, 4, 7, d, 1, 1, 16, ctypes.c_float(0.1), dtype,
                                          None) == want, (d, dtype)
        assert lib.lvamd_paged_attention_merge(None, None, None, 0, 0, None, 1, 4, 7, d, 1, 16, 2, None) == want
        assert (lib.lvamd_paged_prefill_waves_built(2, d, 4) == 1) == (want == -1)
        assert lib.lvamd_paged_prefill_key_tokens(2, d) == (-2 if want == -2 else 64 if d <= 128 else 32)
    assert lib.lvamd_paged_prefill_waves_built(1, 112, 8) == 1 and lib.lvamd_paged_prefill_waves_built(1, 144, 8) == 0
    assert lib.lvamd_paged_decode(None, 0, 0, *no_append, None, None, None, 0, 0, None, None, 1, None, None,
                                  None, None, 0, 4, 7, 128, 1, 1, 16, ctypes.c_float(0.1), 2, None) == -1
    assert lib.lvamd_paged_decode(None, 0, 0, *no_append, None, None, None, 0, 0, None, None, 1, None, None,
                                  None, None, 0, 4, 7, 128, 2, 1, 16, ctypes.c_float(0.1), 2, None) == -2
    # The workgroup split: one column tile, whole workgroups.
    assert lib.lvamd_paged_decode(None, 0, 0, *no_append, None, None, None, 0, 0, None, None, 4, None, None,
                                  None, None, 0, 4, 7, 128, 4, 4, 16, ctypes.c_float(0.1), 2, None) == -2
    assert lib.lvamd_paged_decode(None, 0, 0, *no_append, None, None, None, 0, 0, None, None, 4, None, None,
                                  None, None, 0, 4, 7, 128, 1, 2, 16, ctypes.c_float(0.1), 2, None) == -2
    assert lib.lvamd_paged_decode(None, 0, 0, *no_append, None, None, None, 0, 0, None, None, 6, None, None,
                                  None, None, 0, 4, 7, 128, 1, 8, 16, ctypes.c_float(0.1), 2, None) == -1
    assert lib.lvamd_paged_decode_split_waves(2, 128) == 8 and lib.lvamd_paged_decode_split_waves(2, 256) == 4
    assert lib.lvamd_paged_decode_split_waves(0, 96) == 8 and lib.lvamd_paged_decode_split_waves(0, 128) == 4
    x = ctypes.c_void_p(16)  # (never dereferenced: the checks run first)
    # One layer's call: a null plan is refused; a plan without decode rows or
    # prefill units launches nothing.
    assert lib.lvamd_paged_attention(None, x, 0, 0, *no_append, x, x, x, 0, 0, ctypes.c_float(0.1), None) == -1
    empty = native.AttentionPlan(num_kv_heads=4, group=7, head_size=128, block_size=16, dtype=2)
    assert lib.lvamd_paged_attention(ctypes.byref(empty), x, 0, 0, *no_append, x, x, x, 0, 0,
                                     ctypes.c_float(0.1), None) == 0
    assert native.host().attend(native.attention_entry(), ctypes.addressof(empty), 16, 0, 0, 0, 0, 0, 0, 0, 0,
                                16, 16, 16, 0, 0, 0.1, 0) == 0
    assert lib.lvamd_paged_attention_merge(None, None, None, 0, 0, None, 1, 4, 7, 128, 1, 16, 2, None) == -1
    assert lib.lvamd_paged_attention_merge(None, None, None, 0, 0, None, 1, 4, 7, 128, 17, 16, 2, None) == -2
    for bad_columns in (0, 17):  # the used columns must lie within a slot's 16 * col_tiles
        assert lib.lvamd_paged_attention_merge(None, None, None, 0, 0, None, 1, 4, 7, 128, 1, bad_columns, 2,
                                               None) == -1
    # Prefill: the workgroup shape must be 4 or 8 waves; K without V and
    # misaligned step K/V are refused.
    prefill = lambda nk, nv, waves: lib.lvamd_paged_prefill(  # noqa: E731
        x, 0, 0, nk, 0, 0, nv, 0, 0, x, x, x, 0, 0, x, x, x, 1, None, None, 0, 2, 7, 128, waves, 16,
        ctypes.c_float(0.1), 2, None)
    assert prefill(None, None, 5) == -1
    assert prefill(x, None, 8) == -1
    assert prefill(ctypes.c_void_p(8), x, 4) == -1 and prefill(x, ctypes.c_void_p(24), 8) == -1
    assert lib.lvamd_paged_prefill_waves_built(2, 128, 8) == 1 and lib.lvamd_paged_prefill_waves_built(2, 256, 8) == 0
    assert lib.lvamd_paged_prefill_waves_built(2, 256, 4) == 1 and lib.lvamd_paged_prefill_waves_built(0, 128, 4) == 0
    assert lib.lvamd_kv_append_rotary(None, 0, 0, None, 0, 0, None, 0, 0, None, 0, 0, None, 0, None, 0, None, None,
                                      None, 1, 4, 2, 127, 2, None) == -1  # odd head size
    assert lib.lvamd_hbm_read_probe(None, 16, None, 1, None) == -1
    assert lib.lvamd_paged_prefill_key_tokens(2, 128) == 64 and lib.lvamd_paged_prefill_key_tokens(2, 256) == 32
    assert lib.lvamd_paged_prefill_key_tokens(0, 128) == -2  # no fp32 prefill kernel
    # Tile sizes per kernel; four column tiles only for rows of at most 256 bytes.
    assert lib.lvamd_paged_decode_tile_tokens(2, 128, 1) == 32
    assert lib.lvamd_paged_decode_tile_tokens(2, 128, 4) == 16
    assert lib.lvamd_paged_decode_tile_tokens(2, 256, 1) == 16
    assert lib.lvamd_paged_decode_tile_tokens(2, 256, 4) == -2
    assert lib.lvamd_paged_decode_tile_tokens(0, 64, 4) == 16
    assert lib.lvamd_paged_decode_tile_tokens(0, 128, 4) == -2
    assert native.decode_max_col_tiles(2, 128) == 4 and native.decode_max_col_tiles(2, 256) == 1

def test_backend_refuses_a_cpu_cache() -> None:
    spec = lv.ModelKVCacheSpec((lv.AttentionLayerSpec("attention", 4, 2, 64),))
    with pytest.raises(lv.KVCacheError, match="requires a GPU"):
        lv.PagedKVCache(spec, lv.PagedKVCacheConfig(num_blocks=4, block_size=2))

    class _CpuCache:
        config = lv.PagedKVCacheConfig(num_blocks=4, block_size=2)

    md = lv.PagedAttentionMetadata(block_tables=((0,),), num_computed_tokens=(0,), query_layouts=_layouts(1))
    with pytest.raises(lv.KVCacheError, match="requires a GPU"):
        lv.HipPagedAttentionBackend().create(_CpuCache(), md)


def test_kv_cache_bytes_per_block() -> None:
    spec = lv.ModelKVCacheSpec((lv.AttentionLayerSpec("attention", 2, 2, 4),))
    assert lv.kv_cache_bytes_per_block(spec, block_size=2, dtype=torch.float32) == 128


def _oracle_message(fn, *args, **kwargs):
    try:
        fn(*args, **kwargs)
    except (O.OracleKVCacheError, ValueError) as exc:
        return type(exc).__name__.replace("Oracle", ""), str(exc)
    return None


def _plan_message(fn, *args, **kwargs):
    try:
        fn(*args, **kwargs)
    except (lv.KVCacheError, ValueError) as exc:
        return type(exc).__name__, str(exc)
    return None


@pytest.mark.parametrize("seed", range(90))
def test_native_table_rules_raise_the_oracles_message(seed) -> None:
    """The native block-table check raises exactly the message the oracle's
    restatement of validate_block_tables raises (paged_attention.py:138-172),
    on valid steps, on each kind of mistake (short/long tables, out-of-range
    ids, aliasing within and across requests, readonly sharing at another
    logical index or of a writable block, readonly counts past the prefix),
    and on steps with two mistakes at once, where the rule order decides."""

    rng = np.random.default_rng(seed)
    bs = int(rng.choice([1, 3, 4, 16]))
    batch = int(rng.integers(1, 7))
    shared = int(rng.integers(0, 3))
    computed = [shared * bs + int(rng.integers(0, 40)) for _ in range(batch)]
    reserved = [int(rng.integers(1, 5)) for _ in range(batch)]
    need = [(c + r + bs - 1) // bs for c, r in zip(computed, reserved)]
    pool = [int(x) for x in rng.permutation(sum(need) + 8)]
    prefix, rest, tables = pool[:shared], pool[shared:], []
    for n in need:
        tables.append(list(prefix) + rest[: n - shared])
        rest = rest[n - shared :]
    readonly = [shared] * batch
    num_blocks = len(pool)

    def plant(kind: int) -> None:
        r = int(rng.integers(0, batch))
        if kind == 1:
            tables[r] = tables[r][:-1] or tables[r]
        elif kind == 2:
            tables[r] = tables[r] + [rest[0] if rest else num_blocks - 1]
        elif kind == 3:
            tables[r][-1] = num_blocks + int(rng.integers(0, 3))
        elif kind == 4 and len(tables[r]) > 1:
            tables[r][-1] = tables[r][0]
        elif kind == 5 and batch > 1:
            tables[r][-1] = tables[(r + 1) % batch][-1]
        elif kind == 6 and shared and batch > 1:
            readonly[r] = 0  # a shared block that this request may write
        elif kind == 7:
            readonly[r] = len(tables[r]) + 1
        elif kind == 8 and shared == 2:  # a shared readonly block at another logical index
            tables[r][0], tables[r][1] = tables[r][1], tables[r][0]

    plant(seed % 9)
    if seed >= 45:
        plant(int(rng.integers(1, 9)))
    md = lv.PagedAttentionMetadata(
        block_tables=tuple(tuple(t) for t in tables), num_computed_tokens=tuple(computed),
        query_layouts=tuple(lv.QueryLayout((-1,)) for _ in range(batch)),
        num_reserved_query_tokens=tuple(reserved), num_readonly_prefix_blocks=tuple(readonly),
    )
    expect = _oracle_message(O.validate_block_tables, md.block_tables, computed, reserved, readonly,
                             num_blocks=num_blocks, block_size=bs)
    assert _plan_message(md.validate_block_tables, num_blocks=num_blocks, block_size=bs) == expect
    assert _plan_message(StepPlan, md, block_size=bs, device=CPU, num_blocks=num_blocks) == expect
    assert _plan_message(StepPlan, md, block_size=bs, device=CPU, num_blocks=num_blocks,
                         shapes=_layer_shapes(bs)) == expect


def _layer_shapes(bs: int) -> LayerShapes:
    """Two layer shapes in ``KERNEL_FACTS`` order: grouped queries with the
    four-column-tile decode kernel and both prefill shapes, and a
    one-query-per-head shape without them."""

    return LayerShapes((
        (7, 4, bs, 128, 64, 1, 0, 0, 4, 1, 2048, 32, 1024, 16, 512, 256, 0, 16, 4, 4, 1, 8, 0, 256, 8),
        (1, 8, bs, 256, 64, 0, 0, 0, 1, 0, 2048, 32, 0, 0, 512, 0, 0, 16, 4, 4, 0, 0, 0, 0, 4),
    ))


@pytest.mark.parametrize("small_buffer", (False, True))
@pytest.mark.parametrize("seed", range(8))
def test_one_call_step_plan_equals_the_per_shape_plan(seed, small_buffer, monkeypatch) -> None:
    """``plan_step`` (validation, staging and every layer shape in one native
    call, written into one buffer) gives the same slots, records, tables,
    ancestor rows and work lists as the step facts plus ``layer_work`` per
    shape; with a staging buffer too small at first it grows and plans again."""

    if small_buffer:
        monkeypatch.setattr(Staging, "MIN_ENTRIES", 16)
    rng = np.random.default_rng(500 + seed)
    bs = int(rng.choice([1, 3, 12, 16]))
    md = _random_metadata(rng, batch=int(rng.integers(1, 12)), bs=bs, tree=seed % 2 == 1)
    num_blocks = sum(len(t) for t in md.block_tables) + 5
    shapes = _layer_shapes(bs)
    one = StepPlan(md, block_size=bs, device=CPU, num_blocks=num_blocks, shapes=shapes)
    ref = StepPlan(md, block_size=bs, device=CPU, num_blocks=num_blocks)
    assert one.slots.tolist() == ref.slots.tolist()
    assert one.req_meta.tolist() == ref.req_meta.tolist()
    assert one.tables.tolist() == ref.tables.tolist()[: one.tables.numel()]
    assert one.vis.tolist() == ref.vis.tolist()[: one.vis.numel()]
    counts = ("col_tiles", "prefill_waves", "waves_per_head", "units_per_wave", "num_partial_slots", "num_jobs",
              "merge_columns", "num_prefill_units", "num_prefill_jobs", "num_prefill_partial_slots",
              "prefill_merge_columns", "group_waves")
    for key in shapes.keys:
        a, b = one.layer_work(key), ref.layer_work(key)
        assert [getattr(a, n) for n in counts] == [getattr(b, n) for n in counts]
        for name in ("pieces", "wave_first", "jobs", "prefill_units", "prefill_jobs"):
            x, y = getattr(a, name), getattr(b, name)
            assert (x is None) == (y is None), name
            if x is not None:
                assert x.tolist() == y.tolist(), name
        # Device addresses: every list present has one, inside the upload.
        base, end = one._blob.data_ptr(), one._blob.data_ptr() + 4 * one._blob.numel()
        for ptr, rows in ((a.pieces_ptr, a.pieces), (a.jobs_ptr, a.jobs), (a.units_ptr, a.prefill_units),
                          (a.prefill_jobs_ptr, a.prefill_jobs)):
            assert (ptr is None) == (rows is None)
            if ptr is not None:
                assert base <= ptr and ptr + 4 * rows.numel() <= end and (ptr - base) % 64 == 0
    # A layer shape asked for later is planned on its own, from the records.
    late = (4, 2, bs, 128, 64, 1, 0, 0, 4, 1, 2048, 32, 1024, 16, 512, 256, 0, 16, 4, 4, 1, 8, 1, 128, 4)
    assert one.layer_work(late).num_prefill_units == ref.layer_work(late).num_prefill_units


def test_prefill_shape_choice_follows_the_measured_workloads() -> None:
    """8-wave prefill workgroups for split-K or short units, 4-wave for long
    unsplit units (the kernel notes hold the measurements)."""

    from light_vllm_amd.plan import choose_prefill_waves

    def pick(q_lens, computed, group, slots_per_head=128, wide=True):
        q_lens = np.asarray(q_lens, dtype=np.int64)
        return choose_prefill_waves(q_lens=q_lens, computed=np.asarray(computed, dtype=np.int64),
                                    rows=q_lens * group > 16, group=group, columns=128, key_tokens=64,
                                    slots_per_head=slots_per_head, wide_built=wide)

    assert pick([512] * 8, [3072] * 8, 7) == 4           # long chunks, no split
    assert pick([512] * 8, [0] * 8, 7) == 8              # short units
    assert pick([9] * 32, [2300] * 32, 6, 256) == 8      # C5 tree verification: split
    assert pick([512] * 2, [16384] * 2, 7) == 8          # few units over long history: split
    assert pick([512] * 8, [3072] * 8, 7, 0) == 4        # splitting disabled, long units
    assert pick([9] * 32, [2300] * 32, 6, 256, wide=False) == 4
    assert pick([1] * 8, [100] * 8, 7) == 4              # no prefill rows


def test_compact_slots_known_answer_and_rules() -> None:
    """compact's slot pairs and its table errors (paged_cache.py:269-312) on
    the reference test's case: table (1, 3, 0, 2), computed 2, block size 2,
    retained (0, 2, 4) -> targets (6, 7, 0) (tests/test_paged_attention.py:178-228)."""

    from types import SimpleNamespace

    from light_vllm_amd.paged_cache import compact_slots

    cfg = SimpleNamespace(block_size=2, num_blocks=4)
    kw = dict(num_computed_tokens=2, num_query_tokens=5, num_reserved_query_tokens=5,
              retained_query_indices=(0, 2, 4))
    assert compact_slots(cfg, (1, 3, 0, 2), **kw) == ((6, 0, 4), (6, 7, 0))
    for table, message in (((1, 3, True, 2), "invalid physical block"), ((1, 3, 0, 4), "invalid physical block"),
                           ((1, 3, 1, 2), "aliases a physical block"), ((1, 3, 0), "exactly cover")):
        with pytest.raises(lv.KVCacheError, match=message):
            compact_slots(cfg, table, **kw)


@pytest.mark.parametrize("seed", range(60))
def test_native_compact_rules_raise_the_oracles_message(seed) -> None:
    """compact's rules in the native planner raise what the oracle's
    restatement of PagedKVCache.compact raises (paged_cache.py:276-302), one
    or two planted mistakes at a time, and valid requests give the oracle's
    slot pairs."""

    from types import SimpleNamespace

    from light_vllm_amd.paged_cache import _compact_plan

    rng = np.random.default_rng(700 + seed)
    bs = int(rng.choice([1, 2, 16]))
    computed, queries = int(rng.integers(0, 50)), int(rng.integers(1, 10))
    reserved = queries + int(rng.integers(0, 3))
    readonly = int(rng.integers(0, computed // bs + 1))
    need = (computed + reserved + bs - 1) // bs
    num_blocks = need + 6
    table = [int(x) for x in rng.permutation(num_blocks)[:need]]
    retained = [int(x) for x in rng.permutation(queries)[: int(rng.integers(1, queries + 1))]]
    counts = dict(num_computed_tokens=computed, num_query_tokens=queries, num_reserved_query_tokens=reserved,
                  num_readonly_prefix_blocks=readonly)

    def plant(kind: int) -> None:
        if kind == 1:
            counts["num_computed_tokens"] = -1
        elif kind == 2:
            counts["num_reserved_query_tokens"] = queries - 1
        elif kind == 3:
            retained[0] = True
        elif kind == 4 and len(retained) > 1:
            retained[1] = retained[0]
        elif kind == 5:
            retained[0] = queries
        elif kind == 6:
            table.append(num_blocks - 1)
        elif kind == 7:
            table[0] = num_blocks
        elif kind == 8 and len(table) > 1:
            table[-1] = table[0]
        elif kind == 9:
            counts["num_readonly_prefix_blocks"] = computed // bs + 1

    plant(seed % 10)
    if seed >= 30:
        plant(int(rng.integers(1, 10)))
    pools = [(np.zeros((num_blocks, bs, 1, 1), np.float32), np.zeros((num_blocks, bs, 1, 1), np.float32))]
    expect = _oracle_message(O.compact, pools, tuple(table), retained_query_indices=tuple(retained),
                             num_blocks=num_blocks, block_size=bs, **counts)
    cfg = SimpleNamespace(block_size=bs, num_blocks=num_blocks)
    request = dict(block_ids=tuple(table), retained_query_indices=tuple(retained), **counts)
    got = _plan_message(_compact_plan, cfg, (request,))
    assert got == expect
    if expect is None:
        moved, src, dst = _compact_plan(cfg, (request,))
        slot = lambda pos: table[pos // bs] * bs + pos % bs  # noqa: E731
        pairs = [(slot(computed + i), slot(computed + j)) for j, i in enumerate(retained)]
        assert list(zip(src.tolist(), dst.tolist())) == [p for p in pairs if p[0] != p[1]]
        assert moved.tolist() == [sum(a != b for a, b in pairs)]


def test_compact_reuses_only_tables_the_step_proved() -> None:
    """A compact request whose block table is the very tuple the step's
    metadata listed, after the step's table check passed, skips the id
    checks (in any request order); a tuple the metadata listed but no table
    check proved is checked in full."""

    from light_vllm_amd.paged_cache import PagedKVCacheConfig, _compact_plan

    bs, nb = 4, 64
    tables = ((0, 1, 2), (3, 4, 5), (6, 7, 8, 9))
    computed = (6, 7, 10)
    layouts = tuple(lv.QueryLayout((-1, 0, 0)) for _ in tables)
    md = lv.PagedAttentionMetadata(block_tables=tables, num_computed_tokens=computed, query_layouts=layouts)
    config = PagedKVCacheConfig(num_blocks=nb, block_size=bs, device=CPU)
    requests = [dict(block_ids=t, num_computed_tokens=c, num_query_tokens=3, num_reserved_query_tokens=3,
                     retained_query_indices=(0, 2)) for t, c in zip(md.block_tables, computed)]
    plain = _compact_plan(config, [dict(r, block_ids=list(r["block_ids"])) for r in requests])
    StepPlan(md, block_size=bs, device=CPU, num_blocks=nb)  # the step's table check
    for order in (requests, requests[::-1], requests[1:2]):
        got = _compact_plan(config, order)
        want = _compact_plan(config, [dict(r, block_ids=list(r["block_ids"])) for r in order])
        assert all((a == b).all() for a, b in zip(got, want))
    assert all((a == b).all() for a, b in zip(_compact_plan(config, requests), plain))
    # Flattened by a new metadata object but never proven: an id past the
    # pool must still be caught.
    bad = ((0, 1, 2), (3, 4, 99), (6, 7, 8, 9))
    lv.PagedAttentionMetadata(block_tables=bad, num_computed_tokens=computed, query_layouts=layouts)
    with pytest.raises(lv.KVCacheError, match="invalid physical block"):
        _compact_plan(config, [dict(requests[1], block_ids=bad[1])])


def test_compact_many_batch_rule_and_missing_arguments() -> None:
    from types import SimpleNamespace

    from light_vllm_amd.paged_cache import _compact_plan

    cfg = SimpleNamespace(block_size=2, num_blocks=8)
    req = dict(block_ids=(0, 1), num_computed_tokens=1, num_query_tokens=2, num_reserved_query_tokens=2,
               retained_query_indices=(1,))
    assert _compact_plan(cfg, [req])[0].tolist() == [1]
    with pytest.raises(lv.KVCacheError, match="same slot"):
        _compact_plan(cfg, [req, req])
    with pytest.raises(TypeError, match="needs block_ids"):
        _compact_plan(cfg, [dict(block_ids=(0, 1), num_computed_tokens=1)])


@pytest.mark.parametrize("seed", range(6))
def test_incremental_planner_paths_agree_with_a_fresh_check_every_step(seed) -> None:
    """Decode-like steps: contexts grow, tables take new blocks, some steps
    swap a request, mutate a list row in place, or plant a mistake (an
    appended block already listed elsewhere or twice, one out of range, a
    readonly change, a shrinking table).  Every step, the native flatten
    (which reuses the previous step's values for identical int objects) must
    equal a fresh conversion, and the native table check (which proves an
    append-only step incrementally) must raise exactly the oracle's message."""

    host = native.host()
    proofs0, checks0, reused0, _ = host.counts()
    rng = np.random.default_rng(900 + seed)
    bs, batch = int(rng.choice([1, 4, 16])), 6
    num_blocks = 400
    free = [int(b) for b in rng.permutation(num_blocks)]
    ints = {b: int(str(b)) for b in range(num_blocks + 8)}  # one int object per id, reused every step
    computed = [int(rng.integers(0, 30)) for _ in range(batch)]
    tables = []
    for c in computed:
        tables.append([ints[free.pop()] for _ in range((c + 1 + bs - 1) // bs)])
    readonly = [0] * batch
    for step in range(60):
        for r in range(batch):
            computed[r] += 1
            while len(tables[r]) < (computed[r] + 1 + bs - 1) // bs:
                tables[r].append(ints[free.pop()])
        kind = int(rng.integers(0, 12)) if step % 3 == 2 else 0
        r = int(rng.integers(0, batch))
        rows = [tuple(t) for t in tables]
        if kind == 1:  # an appended block already in another table
            rows[r] = rows[r] + (rows[(r + 1) % batch][-1],)
            computed_step = list(computed)
            computed_step[r] += bs
        elif kind == 2:  # an appended block out of range
            rows[r] = rows[r] + (ints[num_blocks + 3],)
            computed_step = list(computed)
            computed_step[r] += bs
        elif kind == 3:  # an appended block listed twice in its own table
            rows[r] = rows[r] + (rows[r][0],)
            computed_step = list(computed)
            computed_step[r] += bs
        elif kind == 4:  # a readonly prefix appears
            computed_step = list(computed)
            readonly_step = list(readonly)
        elif kind == 5:  # a row given as a list that is mutated in place afterwards
            rows[r] = list(rows[r])
            computed_step = list(computed)
        else:
            computed_step = list(computed)
        readonly_step = list(readonly)
        if kind == 4:
            readonly_step[r] = min(1, computed_step[r] // bs)
        if kind == 6 and len(rows[r]) > 1:  # a shrinking table (coverage breaks)
            rows[r] = rows[r][:-1]
        if kind == 7:  # a request replaced by a fresh one
            fresh = [ints[free.pop()] for _ in range((3 + 1 + bs - 1) // bs)]
            tables[r] = fresh
            computed[r] = computed_step[r] = 3
            rows[r] = tuple(fresh)
        reserved = [1] * batch
        flat, counts, status = host.flatten(rows, False)
        assert status == 0
        expect_flat = [b for row in rows for b in row]
        assert np.frombuffer(flat, dtype=np.int32).tolist() == expect_flat
        assert np.frombuffer(counts, dtype=np.int64).tolist() == [len(row) for row in rows]
        if kind == 5:
            rows[r].append(ints[num_blocks + 1])  # in place: the next flatten must not trust it
            again, _, _ = host.flatten(rows, False)
            assert np.frombuffer(again, dtype=np.int32).tolist() == [b for row in rows for b in row]
            rows[r].pop()
            host.flatten(rows, False)
        expect = _oracle_message(O.validate_block_tables, rows, computed_step, reserved, readonly_step,
                                 num_blocks=num_blocks, block_size=bs)
        rule, _ = host.validate(np.frombuffer(flat, dtype=np.int32), np.frombuffer(counts, dtype=np.int64),
                                np.asarray(computed_step, dtype=np.int64), np.asarray(reserved, dtype=np.int64),
                                np.asarray(readonly_step, dtype=np.int64), num_blocks, bs)
        from light_vllm_amd.facts import TABLE_RULES
        got = None if rule == 0 else ("KVCacheError", TABLE_RULES[rule])
        assert got == expect, f"step {step} kind {kind}"
    proofs, checks, reused, _ = host.counts()
    assert proofs - proofs0 >= 20 and checks - checks0 >= 5, "both table paths must be exercised"
    assert reused - reused0 > 0, "the flatten must have reused the previous step's values"


def _run_ordered(pool: np.ndarray, src, dst, starts, rng) -> None:
    """The one-pass compact's schedule on the CPU: each group moves its pairs
    in batches of 16 (every source of a batch read before its destinations
    are written), batches of one group in order, groups interleaved in a
    random order (the GPU runs them side by side at any relative speed)."""

    nxt = [int(starts[g]) for g in range(starts.size - 1)]
    live = [g for g in range(starts.size - 1) if nxt[g] < starts[g + 1]]
    while live:
        g = live[int(rng.integers(len(live)))]
        b, end = nxt[g], min(nxt[g] + 16, int(starts[g + 1]))
        rows = pool[src[b:end]].copy()
        pool[dst[b:end]] = rows
        nxt[g] = end
        if end == starts[g + 1]:
            live.remove(g)


@pytest.mark.parametrize("seed", range(40))
def test_ordered_compact_schedule_reproduces_the_oracle(seed) -> None:
    """Whenever ordered_groups accepts a step's compact pairs, every
    interleaving of the one-pass kernel's per-group batches leaves the pool
    as the oracle's compact (all sources read before any destination) does;
    steps whose retained indices are strictly increasing are always
    accepted."""

    from types import SimpleNamespace

    from light_vllm_amd.paged_cache import ORDERED_MAX_PAIRS, _compact_plan, ordered_groups

    rng = np.random.default_rng(900 + seed)
    bs = int(rng.choice([1, 3, 16]))
    sorted_only = seed % 2 == 0
    n_req = int(rng.integers(1, 9))
    requests, tables, args_list = [], [], []
    num_blocks = 0
    specs = []
    for _ in range(n_req):
        computed, q = int(rng.integers(0, 40)), int(rng.integers(1, 70))
        keep = int(rng.integers(1, q + 1))
        retained = [int(x) for x in rng.permutation(q)[:keep]]
        if sorted_only:
            retained.sort()
        specs.append((computed, q, tuple(retained)))
        num_blocks += (computed + q + bs - 1) // bs
    num_blocks += 4
    perm = [int(x) for x in rng.permutation(num_blocks)]
    off = 0
    for computed, q, retained in specs:
        need = (computed + q + bs - 1) // bs
        table = tuple(perm[off : off + need])
        off += need
        args = dict(num_computed_tokens=computed, num_query_tokens=q, num_reserved_query_tokens=q,
                    retained_query_indices=retained)
        requests.append(dict(block_ids=table, **args))
        tables.append(table)
        args_list.append(args)
    cfg = SimpleNamespace(block_size=bs, num_blocks=num_blocks)
    moved, src, dst = _compact_plan(cfg, tuple(requests))
    starts = ordered_groups(moved, src, dst)
    if sorted_only and int(moved.max(initial=0)) <= ORDERED_MAX_PAIRS and src.size:
        assert starts is not None, "strictly increasing retained indices must take the one-pass compact"
    pool = rng.standard_normal((num_blocks, bs, 1, 1)).astype(np.float32)
    expect = [(pool.copy(), pool.copy())]
    for table, args in zip(tables, args_list):
        O.compact(expect, table, num_blocks=num_blocks, block_size=bs, **args)
    if starts is None:
        return
    assert starts[0] == 0 and starts[-1] == src.size and np.all(np.diff(starts) > 0)
    for schedule in range(4):
        got = pool.copy()
        _run_ordered(got.reshape(-1), src, dst, starts, np.random.default_rng(schedule))
        np.testing.assert_array_equal(got, expect[0][0])


def test_ordered_groups_refuses_unsafe_orders() -> None:
    """A destination read by a later pair of its group, a row one group
    writes and another reads, and a group past the length cap all take the
    two-phase compact."""

    from light_vllm_amd.paged_cache import ORDERED_MAX_PAIRS, ordered_groups

    i64 = lambda *v: np.array(v, dtype=np.int64)  # noqa: E731
    # Pair 0 writes slot 10, which pair 1 reads afterwards.
    assert ordered_groups(i64(2), i64(13, 10), i64(10, 12)) is None
    # Pair 1 writes slot 13 after pair 0 read it: safe.
    assert ordered_groups(i64(2), i64(13, 14), i64(12, 13)).tolist() == [0, 2]
    # Request 0 writes slot 20, which request 1 reads.
    assert ordered_groups(i64(1, 1), i64(21, 20), i64(20, 30)) is None
    assert ordered_groups(i64(1, 0, 1), i64(21, 31), i64(20, 30)).tolist() == [0, 1, 2]
    n = ORDERED_MAX_PAIRS + 1
    assert ordered_groups(i64(n), np.arange(100, 100 + n), np.arange(n)) is None
    assert ordered_groups(i64(n - 1), np.arange(100, 99 + n), np.arange(n - 1)) is not None


_ATTEND_FN = ctypes.CFUNCTYPE(
    ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
    ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
    ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p,
)


def test_attend_tensors_passes_the_tensors_and_refuses_what_the_fast_path_cannot_take() -> None:
    """forward's native fast path (the host module's attend_tensors), with a
    recording stand-in for lvamd_paged_attention: every pointer, stride,
    scale and stream arrives as given (the layer's pools and output rows
    apart from the shape's facts); each broken rule returns the not-fast
    code without calling it, and a library status comes back."""

    calls = []

    def record(*args):
        calls.append(args)
        return -7 if len(calls) == 3 else 0

    fn = _ATTEND_FN(record)
    fn_addr = ctypes.cast(fn, ctypes.c_void_p).value
    host = native.host()
    not_fast = 1 << 30
    tokens, hq, hkv, d = 5, 8, 2, 64
    dt = torch.bfloat16
    q = torch.zeros((tokens, hq, d), dtype=dt)
    k = torch.zeros((tokens, hkv, d), dtype=dt)
    v = torch.zeros((tokens, hkv, d), dtype=dt)
    shape = (fn_addr, 0x1000, hq * d, d, dt, -1, 2, tokens, hq, hkv, d, lambda dev: 0x5000 + dev)
    pools = (0x2000, 0x3000)
    assert host.attend_tensors(shape, *pools, 0x4000, q, k, v, 0.125) == 0
    got = calls[-1]
    assert got[0] == 0x1000 and got[1] == q.data_ptr() and got[2:4] == (hq * d, d)
    assert got[4] == k.data_ptr() and got[5:7] == (hkv * d, d) and got[7] == v.data_ptr() and got[8:10] == (hkv * d, d)
    assert got[10:13] == (0x2000, 0x3000, 0x4000) and got[13:15] == (hq * d, d)
    assert got[15] == pytest.approx(0.125) and got[16] == 0x5000 - 1
    # Another layer of the shape: its own pools and output rows.
    assert host.attend_tensors(shape, 0x6000, 0x7000, 0x8000, q, k, v, 0.125) == 0
    assert calls[-1][10:13] == (0x6000, 0x7000, 0x8000) and calls[-1][0] == 0x1000
    # Strided rows (a view of a wider buffer) are taken as they are.
    wide = torch.zeros((tokens, hq + 8, d), dtype=dt)[:, 4 : 4 + hq]
    # A library status comes back unchanged (the third call returns -7).
    assert host.attend_tensors(shape, *pools, 0x4000, wide, k, v, 0.5) == -7 and calls[-1][1] == wide.data_ptr()
    assert calls[-1][2:4] == ((hq + 8) * d, d)
    n = len(calls)
    refused = [
        (q.float(), k, v),                                     # dtype
        (q[:, :, :32], k, v),                                  # shape
        (q, k[:4], v),                                         # tokens
        (q.transpose(1, 2).contiguous().transpose(1, 2), k, v),  # last dim not contiguous
        (torch.zeros(tokens * hq * d + 1, dtype=dt)[1:].view(tokens, hq, d), k, v),  # 2-byte offset: unaligned
    ]
    padded = (q, k, torch.zeros((tokens, hkv, d + 8), dtype=dt)[:, :, :d])  # 144-byte rows: still 16-byte aligned
    for args in refused:
        assert host.attend_tensors(shape, *pools, 0x4000, *args, 0.5) == not_fast
    assert len(calls) == n
    assert host.attend_tensors(shape, *pools, 0x4000, *padded, 0.5) == 0
    odd = torch.zeros((tokens, hkv, d + 1), dtype=dt)[:, :, :d]  # 130-byte rows: not 16-byte aligned
    assert host.attend_tensors(shape, *pools, 0x4000, q, k, odd, 0.5) == not_fast
    other_device = shape[:5] + (0,) + shape[6:]
    assert host.attend_tensors(other_device, *pools, 0x4000, q, k, v, 0.5) == not_fast
    with pytest.raises(ValueError):
        host.attend_tensors(shape[:11], *pools, 0x4000, q, k, v, 0.5)
