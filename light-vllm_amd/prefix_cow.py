"""Copy-on-write producer for partial prefix pages (the caller of ``copy_blocks``).

light-vllm's prefix cache shares only complete, committed prompt pages: a
sequence whose prompt matches another's for P tokens reuses the P // bs full
pages and recomputes the P % bs tokens of the partial page
(src/light_vllm/runtime/kv_cache.py:676, :711-723; tails stay private).
This producer lets the partial page be shared too, by copy: the new
sequence takes the donor's full pages as its readonly prefix, a freshly
allocated private page receives a copy of the donor's partial page, and
the new sequence starts with P computed tokens.  Its own writes then go to
its private page only.

Design (the constraints the step's metadata rules put on it):

* Shared pages must be readonly in every sharer at the same logical index
  (``PagedAttentionMetadata.validate_block_tables``, paged_attention.py:
  138-172): the donor must already hold its full shared pages as readonly
  (light-vllm marks published pages readonly, kv_cache.py:711-723), and the
  new table lists them at the same indices with readonly = P // bs.
* The partial page is never shared: the copy gives the new sequence its own
  page at index P // bs, so both sequences may append into it.
* The copy must land before the step's first write into the private page:
  ``PagedKVCache.copy_blocks`` enqueues on the current stream, so calling it
  before ``forward`` is enough (one launch for every copy of the step).
* The copied page's slots at offsets >= P % bs hold the donor's later
  tokens, not the new sequence's: they are positions >= its computed count,
  which attention reads only after this step writes them (write before
  attend), so no stale value is ever read.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Sequence

from light_vllm_amd import errors


@dataclass(frozen=True, slots=True)
class SharedPrefix:
    """One new sequence's start from a donor's first ``num_computed_tokens`` tokens."""

    block_ids: tuple[int, ...]         # the donor's full pages, then the private copy (if any)
    num_readonly_prefix_blocks: int    # the donor's full pages, readonly in both tables
    num_computed_tokens: int           # P: the shared tokens, none recomputed
    copy: tuple[int, int] | None       # (donor's partial page, private page), or None when P % bs == 0


def share_prefix(
    donor_block_ids: Sequence[int],
    donor_readonly_blocks: int,
    shared_tokens: int,
    *,
    block_size: int,
    allocate_block: Callable[[], int],
) -> SharedPrefix:
    """Start a sequence from the first ``shared_tokens`` tokens of a donor.

    ``donor_block_ids`` is the donor's block table (it must cover the shared
    tokens), ``donor_readonly_blocks`` how many of its leading pages are
    readonly; every full page of the shared range must be among them.
    ``allocate_block`` returns a free physical page (the block manager's
    allocator); it is called once, and only when the shared range ends
    inside a page.
    """

    if type(block_size) is not int or block_size <= 0:
        raise ValueError("block size must be a positive integer")
    if type(shared_tokens) is not int or shared_tokens <= 0:
        raise ValueError("shared prefix must be a positive number of tokens")
    table = tuple(donor_block_ids)
    full, partial = divmod(shared_tokens, block_size)
    if len(table) * block_size < shared_tokens:
        raise errors.KVCacheError("donor block table does not cover the shared prefix")
    if type(donor_readonly_blocks) is not int or donor_readonly_blocks < full:
        raise errors.KVCacheError("shared full pages must be readonly in the donor")
    prefix = table[:full]
    if partial == 0:
        return SharedPrefix(prefix, full, shared_tokens, None)
    private = allocate_block()
    if type(private) is not int or private < 0 or private in table:
        raise errors.KVCacheError("allocated page must be a free physical page")
    return SharedPrefix(prefix + (private,), full, shared_tokens, (table[full], private))


def copy_commands(starts: Sequence[SharedPrefix]) -> tuple[tuple[int, ...], tuple[int, ...]]:
    """(sources, destinations) of every page copy of one step's new sequences,
    for a single ``PagedKVCache.copy_blocks`` call before the step's forward."""

    pairs = [s.copy for s in starts if s.copy is not None]
    return tuple(p[0] for p in pairs), tuple(p[1] for p in pairs)
