"""The copy-on-write producer for partial prefix pages (CPU): its tables,
readonly counts and copy commands, the metadata rules they satisfy (and
that sharing the partial page without a copy breaks), and, through the
oracle, that a copied start attends exactly like its donor's prefix."""

from __future__ import annotations

import numpy as np
import pytest

import light_vllm_amd as lv
from oracle import paged_kv_oracle as O


def _allocator(free):
    free = list(free)
    return lambda: free.pop(0)


def test_partial_page_is_copied_full_pages_shared() -> None:
    start = lv.share_prefix((10, 11, 12, 13), 3, 40, block_size=16, allocate_block=_allocator([50]))
    assert start == lv.SharedPrefix((10, 11, 50), 2, 40, (12, 50))
    whole = lv.share_prefix((10, 11, 12, 13), 2, 32, block_size=16, allocate_block=_allocator([]))
    assert whole == lv.SharedPrefix((10, 11), 2, 32, None)  # no allocation when the range ends on a page
    first = lv.share_prefix((7,), 0, 5, block_size=16, allocate_block=_allocator([9]))
    assert first == lv.SharedPrefix((9,), 0, 5, (7, 9))
    assert lv.copy_commands([start, whole, first]) == ((12, 7), (50, 9))


def test_producer_rules() -> None:
    with pytest.raises(lv.KVCacheError, match="readonly in the donor"):
        lv.share_prefix((10, 11, 12), 1, 40, block_size=16, allocate_block=_allocator([50]))
    with pytest.raises(lv.KVCacheError, match="does not cover"):
        lv.share_prefix((10, 11), 2, 40, block_size=16, allocate_block=_allocator([50]))
    with pytest.raises(lv.KVCacheError, match="free physical page"):
        lv.share_prefix((10, 11, 12), 2, 40, block_size=16, allocate_block=_allocator([12]))
    with pytest.raises(ValueError, match="positive number of tokens"):
        lv.share_prefix((10,), 0, 0, block_size=16, allocate_block=_allocator([50]))
    with pytest.raises(ValueError, match="block size"):
        lv.share_prefix((10,), 0, 3, block_size=0, allocate_block=_allocator([50]))


def _step(bs: int, shared: int, rng):
    """A donor with ``shared + 20`` computed tokens and three sequences started
    from its first ``shared`` tokens, each verifying a draft tree."""

    donor_computed = shared + 20
    donor = tuple(range(-(-(donor_computed + 1) // bs)))
    readonly = shared // bs
    nxt = [len(donor)]

    def alloc():
        nxt[0] += 1
        return nxt[0] - 1

    starts = [lv.share_prefix(donor, readonly, shared, block_size=bs, allocate_block=alloc) for _ in range(3)]
    tables, computed, layouts = [donor], [donor_computed], [lv.linear_query_layout(1)]
    for s in starts:
        parents = tuple([-1] + [int(rng.integers(0, i)) for i in range(1, 7)])
        need = -(-(s.num_computed_tokens + len(parents)) // bs)
        extra = []
        while len(s.block_ids) + len(extra) < need:
            extra.append(alloc())
        tables.append(s.block_ids + tuple(extra))
        computed.append(s.num_computed_tokens)
        layouts.append(lv.QueryLayout(parents))
    ro = (readonly,) + tuple(s.num_readonly_prefix_blocks for s in starts)
    md = lv.PagedAttentionMetadata(block_tables=tuple(tables), num_computed_tokens=tuple(computed),
                                   query_layouts=tuple(layouts), num_readonly_prefix_blocks=ro)
    return md, starts, nxt[0]


@pytest.mark.parametrize("bs,shared", ((16, 40), (16, 48), (12, 100), (3, 7), (1, 9)))
def test_copied_start_passes_the_table_rules_and_attends_like_the_donor(bs, shared) -> None:
    rng = np.random.default_rng(bs * 100 + shared)
    md, starts, num_blocks = _step(bs, shared, rng)
    md.validate_block_tables(num_blocks=num_blocks, block_size=bs)
    if shared % bs:
        # Sharing the partial page itself, without the copy, breaks the rule
        # that shared pages are readonly in every sharer.
        naive = list(md.block_tables)
        naive[1] = md.block_tables[0][: shared // bs + 1] + md.block_tables[1][shared // bs + 1 :]
        bad = lv.PagedAttentionMetadata(block_tables=tuple(naive), num_computed_tokens=md.num_computed_tokens,
                                        query_layouts=md.query_layouts,
                                        num_readonly_prefix_blocks=md.num_readonly_prefix_blocks)
        with pytest.raises(lv.KVCacheError, match="alias a physical block across requests"):
            bad.validate_block_tables(num_blocks=num_blocks, block_size=bs)
    # Oracle: random pools, the copies by block_copy's closed form, then each
    # started sequence's tree over its own table equals the same queries over
    # the donor's table for the shared tokens.
    h, d = 2, 16
    kp = rng.standard_normal((num_blocks, bs, h, d)).astype(np.float32)
    vp = rng.standard_normal((num_blocks, bs, h, d)).astype(np.float32)
    src, dst = lv.copy_commands(starts)
    before_k, before_v = kp.copy(), vp.copy()
    O.block_copy([(kp, vp)], src, dst)
    changed = sorted(set(np.flatnonzero((kp != before_k).any(axis=(1, 2, 3))).tolist()))
    assert set(changed) <= set(dst) and all((kp[t] == before_k[s]).all() and (vp[t] == before_v[s]).all()
                                           for s, t in zip(src, dst))
    for r in range(1, len(md.block_tables)):
        layout = md.query_layouts[r].parent_indices
        q = rng.standard_normal((len(layout), 2 * h, d)).astype(np.float32)
        # This step's tokens are written to the sequence's own slots first.
        slots = O.slot_mapping([md.block_tables[r]], [md.num_computed_tokens[r]], [len(layout)], [len(layout)], bs)
        knew = rng.standard_normal((len(layout), h, d)).astype(np.float32)
        vnew = rng.standard_normal((len(layout), h, d)).astype(np.float32)
        O.append(kp, vp, knew, vnew, slots)
        got = O.paged_attention(q, kp, vp, [md.block_tables[r]], [shared], [layout], scale=0.25)
        # The same attention with the shared tokens read from the donor's pages:
        # a table whose leading pages are the donor's up to the partial page.
        mixed = md.block_tables[0][: -(-shared // bs)] + md.block_tables[r][-(-shared // bs) :]
        kd, vd = kp.copy(), vp.copy()
        O.append(kd, vd, knew, vnew, O.slot_mapping([mixed], [shared], [len(layout)], [len(layout)], bs))
        want = O.paged_attention(q, kd, vd, [mixed], [shared], [layout], scale=0.25)
        np.testing.assert_allclose(got, want, rtol=0, atol=1e-6)
