"""Host-side step plan: everything the kernels need, built once per model step.

light-vllm builds its per-step device metadata in ``TritonPagedAttention.__init__``
(src/light_vllm/runtime/execution/triton_paged_attention.py:402-448): block
tables padded to the longest request, computed counts, query lengths, query
starts and request indices, staged through one pinned H2D copy
(src/light_vllm/runtime/execution/cuda_staging.py:27-49).  This plan carries
the same facts in a ragged layout the gfx950 kernels read directly:

* ``slots``    int64 [T]   physical slot of every packed query token
  (``PagedAttentionMetadata.slot_mapping``, paged_attention.py:110-136);
* ``req_meta`` int32 [B, 8] (table_off, num_blocks, computed, q_len, q_start,
  vis_off, vis_words, 0);
* ``tables``   int32 flat concatenation of the block tables (no padding);
* ``vis``      uint32 ancestor bitmask rows for non-linear (tree) requests,
  bit j of row q set iff query q sees query j (``visibility_tensor``,
  paged_attention.py:174-186, packed 32 to a word);
* per (group size, kv heads): the stream-K split of the decode rows (pieces,
  each wave's first piece, merge jobs) and query blocks for the prefill rows.

All int32 facts of a step share one pinned buffer and one non-blocking H2D
copy on the current stream; the work lists of each group size add one more.
"""

from __future__ import annotations

import itertools
from collections import OrderedDict
from dataclasses import dataclass

import numpy as np
import torch
from torch import Tensor

from light_vllm_amd.errors import KVCacheError
from light_vllm_amd.layout import is_linear, query_visibility

# Requests whose queries x group fit one 16-column MFMA tile use the split-K
# decode kernel; wider ones (prompt chunks, tree verification) use the MFMA
# prefill kernel when it covers the layer's shape, whose four waves share
# each K/V tile.
DECODE_MAX_COLUMNS = 16
# Smallest key range (in prefill key tiles) the planner gives one prefill
# workgroup when it splits units to fill the GPU.
PREFILL_MIN_TILES = 4
# Compute units of an MI355X; the planner aims for several waves per CU.
NUM_CUS = 256
# Block-table entries a decode partition may span (the kernel's LDS slice).
TABLE_SLICE = 256


PIECE_FIELDS = 16
PREFILL_FIELDS = 8
PIECE_BLOCKS = 5  # first-tile block ids carried in piece fields 11..15
MERGE_FIELDS = 8
# Default stream-K granularity: shares and piece boundaries fall on multiples
# of this many tokens.  The backend passes the decode kernel's own tile size
# instead, so that every piece is whole tiles (a partial tile costs a full
# load round trip; measured on C2, 16-token units were slower than 32).
UNIT_TOKENS = 32
# Relative cost per K/V token of the four-column-tile decode kernel against
# the one-tile kernel (16-token tiles and four accumulator sets).  The
# planner uses four column tiles per wave when
#   sum(seq * ceil(tiles / 4)) * COL_TILES4_COST < sum(seq * tiles)
# over the decode rows, i.e. when the K/V re-reads it saves outweigh its
# slower tiles.  Measured on a C5-shaped layer (bf16, D = 128, 4 column
# tiles per request): 39.9 us at four tiles per wave against 47.5 us at one,
# i.e. 4 x 39.9 / 47.5 = 3.4 per token.
COL_TILES4_COST = 3.4

_BIT_WEIGHTS = (np.uint64(1) << np.arange(32, dtype=np.uint64)).astype(np.uint64)


def stream_k_pieces(
    *,
    seq: np.ndarray,
    ngroups: np.ndarray,
    rows: np.ndarray,
    req_meta: np.ndarray,
    flat_tables: np.ndarray,
    num_kv_heads: int,
    resident_waves: int,
    block_size: int,
    min_units_per_wave: int = 4,
    max_units_per_wave: int | None = None,
    unit_tokens: int = UNIT_TOKENS,
):
    """Split the decode work evenly over the waves the GPU holds at once.

    A segment is one (request, column group), a column group being the
    ``col_tiles`` column tiles one decode wave computes together (``ngroups``
    per request); it has ceil(seq / unit_tokens) units.  The segments of all decode rows are laid end to end and the
    flattened unit range is cut into ``waves_per_head`` contiguous shares
    that differ by at most one unit (the same cut for every kv head).  A wave's share is a list of
    pieces: the part of each segment it covers.  A piece that covers a whole
    segment writes the output directly; otherwise it writes a partial
    (max, sum, acc) to its slot and a merge job combines the segment's
    partials.  Returns (pieces [n, 16] int64, wave_first [W + 1], W, largest
    share, jobs [m, 8] = (req, column group, first slot, partials, q_start,
    q_len, 0, 0), num_slots).
    """

    seg_req = np.repeat(np.flatnonzero(rows), ngroups[rows])
    seg_group = np.concatenate([np.arange(n) for n in ngroups[rows]]) if rows.any() else np.zeros(0, np.int64)
    seg_tiles = -(-seq[seg_req] // unit_tokens)
    total = int(seg_tiles.sum())
    seg_start = np.zeros(len(seg_req) + 1, dtype=np.int64)
    np.cumsum(seg_tiles, out=seg_start[1:])
    # The block-table slice of a piece must fit the kernel's LDS copy.
    cap = max(1, ((TABLE_SLICE - 2) * block_size) // unit_tokens)
    if max_units_per_wave is not None:
        cap = max(1, min(cap, max_units_per_wave))
    waves = max(1, min(max(1, resident_waves // num_kv_heads), -(-total // min_units_per_wave)))
    waves = max(waves, -(-total // cap))
    per_wave = -(-total // waves)  # the largest share; never above cap
    # As few waves as give that largest share: every wave then carries a
    # full share (C2: 237 waves per head of 10 tiles, not 256 of 9 or 10),
    # so the memory system stays busy until the end and no wave runs a
    # lone extra tile after the others finish.
    if per_wave:
        waves = -(-total // per_wave)
    # Balanced shares: wave w covers units [w * total // W, (w + 1) * total // W),
    # so shares differ by at most one unit and every wave has work.
    bounds = (np.arange(waves + 1, dtype=np.int64) * total) // waves
    cuts = np.unique(np.concatenate((seg_start, bounds)))
    lo, hi = cuts[:-1], cuts[1:]
    seg = np.searchsorted(seg_start, lo, side="right") - 1
    wave = np.searchsorted(bounds, lo, side="right") - 1
    npieces = np.bincount(seg, minlength=len(seg_req))
    multi = npieces[seg] > 1
    slot = np.where(multi, np.cumsum(multi) - 1, -1)
    req = seg_req[seg]
    pieces = np.zeros((len(lo), PIECE_FIELDS), dtype=np.int64)
    pieces[:, 0] = req
    pieces[:, 1] = seg_group[seg]
    pieces[:, 2] = (lo - seg_start[seg]) * unit_tokens
    pieces[:, 3] = np.minimum((hi - seg_start[seg]) * unit_tokens, seq[req])
    pieces[:, 4] = slot
    pieces[:, 5] = req_meta[req, 0]  # table_off
    pieces[:, 6] = req_meta[req, 2]  # computed
    pieces[:, 7] = req_meta[req, 3]  # q_len
    pieces[:, 8] = req_meta[req, 4]  # q_start
    pieces[:, 9] = req_meta[req, 5]  # vis_off
    pieces[:, 10] = req_meta[req, 6]  # vis_words
    # Physical ids of each piece's first PIECE_BLOCKS logical blocks (0 past
    # the request's table): the kernel issues the first tile from them.
    lb0 = pieces[:, 2] // block_size
    nblk = req_meta[req, 1]
    j = np.arange(PIECE_BLOCKS)
    ok = lb0[:, None] + j[None, :] < nblk[:, None]
    idx = np.where(ok, req_meta[req, 0][:, None] + lb0[:, None] + j[None, :], 0)
    pieces[:, 11 : 11 + PIECE_BLOCKS] = np.where(ok, flat_tables[idx] if flat_tables.size else 0, 0)
    wave_first = np.searchsorted(wave, np.arange(waves + 1), side="left")
    first = multi & (lo == seg_start[seg])
    jreq = req[first]
    jobs = np.zeros((int(first.sum()), MERGE_FIELDS), dtype=np.int64)
    jobs[:, 0] = jreq
    jobs[:, 1] = seg_group[seg[first]]
    jobs[:, 2] = slot[first]
    jobs[:, 3] = npieces[seg[first]]
    jobs[:, 4] = req_meta[jreq, 4]  # q_start
    jobs[:, 5] = req_meta[jreq, 3]  # q_len
    return pieces, wave_first, waves, per_wave, jobs, int(multi.sum())


PREFILL_WIDE_MAX_TILES = 20  # mean key tiles per unit up to which 8-wave prefill workgroups win


def choose_prefill_waves(
    *, q_lens: np.ndarray, computed: np.ndarray, rows: np.ndarray, group: int, columns: int, key_tokens: int,
    slots_per_head: int, wide_built: bool,
) -> int:
    """Workgroup shape of the prefill kernel for these rows: 8 waves of one
    column tile when the units will be split over the resident workgroups or
    are short (mean key tiles per unit at most PREFILL_WIDE_MAX_TILES), where
    latency hiding pays; else 4 waves of two column tiles, whose K/V LDS reads
    each feed two MFMAs.  Measured per workload in the prefill kernel's notes.
    """

    if not wide_built or not rows.any():
        return 4
    ncols = q_lens * group
    nunit = np.where(rows, -(-ncols // columns), 0)
    n = int(nunit.sum())
    req = np.repeat(np.arange(len(q_lens)), nunit)
    starts = np.zeros(len(q_lens), dtype=np.int64)
    np.cumsum(nunit[:-1], out=starts[1:])
    col0 = (np.arange(n) - starts[req]) * columns
    last = np.minimum(col0 + columns, ncols[req]) - 1
    tiles = -(-(computed[req] + last // group + 1) // key_tokens)
    split = bool(slots_per_head) and n < slots_per_head
    return 8 if split or float(tiles.mean()) <= PREFILL_WIDE_MAX_TILES else 4


def prefill_pieces(
    *,
    q_lens: np.ndarray,
    computed: np.ndarray,
    rows: np.ndarray,
    req_meta: np.ndarray,
    group: int,
    columns: int,
    key_tokens: int,
    slots_per_head: int,
    min_tiles: int = PREFILL_MIN_TILES,
):
    """Prefill work units of the ``rows`` requests, split over keys when the
    units alone cannot fill the GPU.

    A unit is up to ``columns`` MFMA columns (query, head-in-group pairs) of
    one request; it needs the keys up to its last query, ceil(kneed /
    key_tokens) tiles.  When there are fewer units than ``slots_per_head``
    (resident prefill workgroups per kv head), every unit's tile range is cut
    into near-equal pieces of at least ``min_tiles`` tiles so that all slots
    get work; the pieces of a split unit write partials (consecutive slots)
    and one merge job per unit combines them.  Returns (units [n, 8] int64,
    heaviest first, as (req, first column, columns, key_begin, key_end, slot,
    0, 0); merge jobs [m, 8] as (req, column group, first slot, pieces,
    q_start, q_len, 0, 0); number of partial slots).
    """

    ncols = q_lens * group
    nunit = np.where(rows, -(-ncols // columns), 0)
    n = int(nunit.sum())
    req = np.repeat(np.arange(len(q_lens)), nunit)
    starts = np.zeros(len(q_lens), dtype=np.int64)
    np.cumsum(nunit[:-1], out=starts[1:])
    col0 = (np.arange(n) - starts[req]) * columns
    cols = np.minimum(columns, ncols[req] - col0)
    kneed = computed[req] + (col0 + cols - 1) // group + 1
    tiles = -(-kneed // key_tokens)
    npieces = np.ones(n, dtype=np.int64)
    if slots_per_head and n < slots_per_head:
        target = max(min_tiles, -(-int(tiles.sum()) // slots_per_head))
        npieces = np.maximum(1, -(-tiles // target))
    total = int(npieces.sum())
    unit = np.repeat(np.arange(n), npieces)
    pstart = np.zeros(n, dtype=np.int64)
    np.cumsum(npieces[:-1], out=pstart[1:])
    i = np.arange(total) - pstart[unit]
    t0 = (i * tiles[unit]) // npieces[unit]
    t1 = ((i + 1) * tiles[unit]) // npieces[unit]
    split = npieces[unit] > 1
    slot = np.where(split, np.cumsum(split) - 1, -1)
    ptab = np.zeros((total, PREFILL_FIELDS), dtype=np.int64)
    ptab[:, 0] = req[unit]
    ptab[:, 1] = col0[unit]
    ptab[:, 2] = cols[unit]
    ptab[:, 3] = t0 * key_tokens
    ptab[:, 4] = np.where(i + 1 < npieces[unit], t1 * key_tokens, 0)
    ptab[:, 5] = slot
    # Heaviest first (keys x columns): better tail balance.
    work = (t1 - t0) * cols[unit]
    order = np.argsort(-work, kind="stable")
    first = split & (i == 0)
    ju = unit[first]
    jobs = np.zeros((int(first.sum()), MERGE_FIELDS), dtype=np.int64)
    jobs[:, 0] = req[ju]
    jobs[:, 1] = col0[ju] // columns
    jobs[:, 2] = slot[first]
    jobs[:, 3] = npieces[ju]
    jobs[:, 4] = req_meta[req[ju], 4]  # q_start
    jobs[:, 5] = req_meta[req[ju], 3]  # q_len
    return ptab[order], jobs, int(split.sum())


# Block tables already proven to hold unique int ids in [0, num_blocks):
# id(table) -> (table, num_blocks).  An entry holds its tuple, so the id
# cannot pass to another object while it is listed, and a tuple of ints
# cannot change, so a listed table needs no second pass.  compact() consults
# it for the tables that the step's attention context has already checked.
# The list keeps its tables alive, so it is bounded to about one step's
# requests; a table that fell out is simply checked again.
_PROVEN_TABLES: "OrderedDict[int, tuple[tuple, int]]" = OrderedDict()
_PROVEN_LIMIT = 256


def note_proven_tables(tables, num_blocks: int) -> None:
    """Record tables that passed the block-table rules for ``num_blocks``
    (their ids are ints, as the metadata constructor requires)."""

    for table in tables:
        if type(table) is tuple:
            _PROVEN_TABLES[id(table)] = (table, num_blocks)
            _PROVEN_TABLES.move_to_end(id(table))
    while len(_PROVEN_TABLES) > _PROVEN_LIMIT:
        _PROVEN_TABLES.popitem(last=False)


def table_proven(table, num_blocks: int) -> bool:
    entry = _PROVEN_TABLES.get(id(table))
    return entry is not None and entry[0] is table and entry[1] == num_blocks


def tables_valid(
    flat: np.ndarray,
    counts: np.ndarray,
    computed: np.ndarray,
    reserved: np.ndarray,
    readonly: np.ndarray,
    *,
    num_blocks: int,
    block_size: int,
) -> bool:
    """Whether ``PagedAttentionMetadata.validate_block_tables`` would pass
    (paged_attention.py:138-173), checked with array passes over the flat
    tables instead of a Python loop per block id:

    * every table has exactly ceil((computed + reserved) / block_size) blocks;
    * every id is < num_blocks;
    * readonly prefix blocks fit the table and the computed prefix;
    * no id repeats within a table;
    * an id shared by several tables sits at the same logical index and is
      in the readonly prefix of every one of them.
    """

    if len(counts) == 0:
        return True
    required = (computed + reserved + block_size - 1) // block_size
    if np.any(counts != required):
        return False
    if flat.size and (int(flat.max()) >= num_blocks or int(flat.min()) < 0):
        return False
    if np.any((readonly > counts) | (readonly * block_size > computed)):
        return False
    if flat.size == 0:
        return True
    uses = np.bincount(flat, minlength=num_blocks)
    if int(uses.max()) <= 1:
        return True  # no id appears twice anywhere
    # Only the ids that repeat need the per-occurrence checks.
    rep = np.flatnonzero(uses[flat] > 1)
    req = np.searchsorted(np.cumsum(counts), rep, side="right")
    starts = np.zeros(len(counts), dtype=np.int64)
    np.cumsum(counts[:-1], out=starts[1:])
    logical = rep - starts[req]
    ro = logical < readonly[req]
    order = np.lexsort((req, flat[rep]))  # by block id, then request
    b, r, lg, o = flat[rep][order], req[order], logical[order], ro[order]
    same = b[1:] == b[:-1]
    if np.any(same & (r[1:] == r[:-1])):
        return False  # repeated within one table
    # Across tables: every occurrence of a shared id (each one after the
    # first compared with the previous) at the same logical index, readonly.
    return not np.any(same & ((lg[1:] != lg[:-1]) | ~o[1:] | ~o[:-1]))


def _stage_int32(array: np.ndarray, device: torch.device) -> Tensor:
    """One pinned host buffer, one non-blocking copy on the current stream."""

    host = torch.from_numpy(np.ascontiguousarray(array, dtype=np.int32))
    if device.type == "cuda":
        host = host.pin_memory()
    return host.to(device, non_blocking=True)


def _job_columns(jobs: np.ndarray, group: int, per_slot: int) -> int:
    """Most columns any merge job covers: its query run times the group, past
    the columns of earlier column groups, at most a slot's columns.  Jobs are
    (req, column group, first slot, partials, q_start, q_len, 0, 0)."""

    cols = np.minimum(per_slot, jobs[:, 5] * group - jobs[:, 1] * per_slot)
    return int(max(1, cols.max()))


@dataclass(frozen=True, slots=True)
class DecodeWork:
    pieces: Tensor | None  # int32 [n_pieces, 16]
    wave_first: Tensor | None  # int32 [waves_per_head + 1]
    waves_per_head: int
    jobs: Tensor | None  # int32 [n_jobs, 8]
    num_jobs: int
    num_partial_slots: int
    units_per_wave: int
    col_tiles: int  # column tiles per decode wave (partials hold 16 * col_tiles columns)
    prefill_units: Tensor | None  # int32 [n_prefill_units, 8]
    num_prefill_units: int
    prefill_jobs: Tensor | None = None  # int32 [n, 8] merge jobs of split prefill units
    num_prefill_jobs: int = 0
    num_prefill_partial_slots: int = 0
    prefill_waves: int = 4  # prefill workgroup shape: 4 waves x 2 column tiles or 8 x 1
    merge_columns: int = 1  # most columns any decode merge job has
    prefill_merge_columns: int = 1  # most columns any prefill merge job has


class StepPlan:
    """Device-resident metadata of one model step (valid for all of its layers)."""

    def __init__(
        self,
        metadata,
        *,
        block_size: int,
        device: torch.device,
        partition_tokens: int | None = None,
        num_blocks: int | None = None,
    ) -> None:
        """With ``num_blocks`` the block tables are validated first, with the
        rules and messages of ``PagedAttentionMetadata.validate_block_tables``
        (paged_attention.py:138-173): a vectorised check over the flat tables,
        and the metadata's own method to raise the exact error when it fails."""

        self.block_size = block_size
        self.device = device
        layouts = tuple(metadata.query_layouts)
        tables = tuple(metadata.block_tables)
        batch = len(tables)
        counts = np.fromiter((len(t) for t in tables), dtype=np.int64, count=batch)
        flat = np.fromiter(itertools.chain.from_iterable(tables), dtype=np.int64, count=int(counts.sum()))
        table_off = np.zeros(batch, dtype=np.int64)
        np.cumsum(counts[:-1], out=table_off[1:])
        computed = np.asarray(metadata.num_computed_tokens, dtype=np.int64)
        if num_blocks is not None and not tables_valid(
            flat, counts, computed, np.asarray(metadata.num_reserved_query_tokens, dtype=np.int64),
            np.asarray(metadata.num_readonly_prefix_blocks, dtype=np.int64), num_blocks=num_blocks,
            block_size=block_size,
        ):
            metadata.validate_block_tables(num_blocks=num_blocks, block_size=block_size)
            # Only a negative id gets here (the metadata constructor rejects them).
            raise KVCacheError("block table contains an out-of-range physical block")
        if num_blocks is not None:
            note_proven_tables(tables, num_blocks)
        q_lens = np.fromiter((len(layout) for layout in layouts), dtype=np.int64, count=batch)
        q_start = np.zeros(batch, dtype=np.int64)
        np.cumsum(q_lens[:-1], out=q_start[1:])
        num_tokens = int(q_lens.sum())

        vis_off = np.full(batch, -1, dtype=np.int64)
        vis_words = np.zeros(batch, dtype=np.int64)
        vis_parts: list[np.ndarray] = []
        running = 0
        for r, layout in enumerate(layouts):
            if is_linear(layout):
                continue
            q = len(layout)
            words = (q + 31) // 32
            rows = np.asarray(query_visibility(layout), dtype=bool)
            padded = np.zeros((q, words * 32), dtype=np.uint64)
            padded[:, :q] = rows
            # bit b of word w of row i  <->  query 32*w + b is visible from query i
            packed = padded.reshape(q, words, 32) @ _BIT_WEIGHTS
            vis_parts.append(packed.astype(np.uint32).reshape(-1))
            vis_off[r] = running
            vis_words[r] = words
            running += q * words
        vis = np.concatenate(vis_parts) if vis_parts else np.zeros(1, dtype=np.uint32)

        req_idx = np.repeat(np.arange(batch), q_lens)
        positions = computed[req_idx] + (np.arange(num_tokens) - q_start[req_idx])
        slots = flat[table_off[req_idx] + positions // block_size] * block_size + positions % block_size

        req_meta = np.zeros((batch, 8), dtype=np.int64)
        req_meta[:, 0] = table_off
        req_meta[:, 1] = counts
        req_meta[:, 2] = computed
        req_meta[:, 3] = q_lens
        req_meta[:, 4] = q_start
        req_meta[:, 5] = vis_off
        req_meta[:, 6] = vis_words
        if flat.size and int(flat.max()) > np.iinfo(np.int32).max:
            raise ValueError("block ids must fit in int32")

        # One int32 blob: [slots as int32 pairs | req_meta | tables | vis].
        parts = [
            slots.astype(np.int64).view(np.int32),
            req_meta.astype(np.int32).reshape(-1),
            flat.astype(np.int32) if flat.size else np.zeros(1, dtype=np.int32),
            vis.view(np.int32),
        ]
        sizes = [p.size for p in parts]
        offs = np.concatenate(([0], np.cumsum(sizes)))
        blob = _stage_int32(np.concatenate(parts), device)
        self.slots = blob[offs[0] : offs[1]].view(torch.int64)
        self.req_meta = blob[offs[1] : offs[2]]
        self.tables = blob[offs[2] : offs[3]]
        self.vis = blob[offs[3] : offs[4]]
        self._blob = blob
        self.num_tokens = num_tokens
        self.batch_size = batch
        self.has_tree = bool(vis_parts)
        self.partition_tokens = partition_tokens

        self._computed = computed
        self._q_lens = q_lens
        self._req_meta = req_meta
        self._flat = flat
        self._work: dict[tuple[int, ...], DecodeWork] = {}
        self._col_tiles: dict[tuple[int, int, int], int] = {}
        # Bound launch arguments per layer shape, filled by the backend.
        self.launches: dict[tuple, object] = {}

    @property
    def num_query_tokens(self) -> int:
        return self.num_tokens

    # -- work lists ---------------------------------------------------------
    def decode_rows(self, prefill_columns: int, group: int = 1) -> np.ndarray:
        """Requests the decode kernel serves (all of them without a prefill kernel)."""

        if prefill_columns > 0:
            return self._q_lens * group <= DECODE_MAX_COLUMNS
        return np.ones(self.batch_size, dtype=bool)

    def choose_col_tiles(self, group: int, prefill_columns: int, max_col_tiles: int) -> int:
        """Column tiles per decode wave for layers with this group size: 4 when
        the decode rows' K/V re-reads at one tile per wave cost more than the
        four-tile kernel's slower tiles (``COL_TILES4_COST``), else 1."""

        if max_col_tiles < 4:
            return 1
        key = (group, prefill_columns, max_col_tiles)
        found = self._col_tiles.get(key)
        if found is None:
            found = self._col_tiles[key] = self._choose_col_tiles(group, prefill_columns)
        return found

    def _choose_col_tiles(self, group: int, prefill_columns: int) -> int:
        rows = self.decode_rows(prefill_columns, group)
        seq = (self._computed + self._q_lens)[rows]
        nct = -(-(self._q_lens[rows] * group) // 16)
        one = float((seq * nct).sum())
        four = float((seq * -(-nct // 4)).sum()) * COL_TILES4_COST
        return 4 if four < one else 1

    def work(
        self, group: int, num_kv_heads: int, resident_waves: int = 8 * NUM_CUS, prefill_columns: int = 0,
        unit_tokens: int = UNIT_TOKENS, col_tiles: int = 1, prefill_key_tokens: int = 64,
        prefill_resident: int = 0, prefill_waves: int = 4,
    ) -> DecodeWork:
        """Work lists for layers of this (group, kv heads) shape.

        ``resident_waves`` is how many decode waves the GPU holds at once,
        ``prefill_columns`` the prefill kernel's unit width (0: every request
        goes through the decode kernel), ``unit_tokens`` the decode kernel's
        tile and ``col_tiles`` its column tiles per wave; ``prefill_key_tokens``
        is the prefill kernel's key tile and ``prefill_resident`` how many
        prefill workgroups of shape ``prefill_waves`` the GPU holds (0: never
        split prefill units).  The library reports the kernel figures per
        dtype and head size.
        """

        key = (group, num_kv_heads, resident_waves, prefill_columns, unit_tokens, col_tiles, prefill_key_tokens,
               prefill_resident, prefill_waves)
        found = self._work.get(key)
        if found is None:
            found = self._build_work(group, num_kv_heads, resident_waves, prefill_columns, unit_tokens, col_tiles,
                                     prefill_key_tokens, prefill_resident, prefill_waves)
            self._work[key] = found
        return found

    def prefill_waves(self, group: int, num_kv_heads: int, prefill_columns: int, prefill_key_tokens: int,
                      prefill_resident: int, wide_built: bool) -> int:
        """The prefill workgroup shape (4 or 8 waves) for this step's wide rows."""

        rows = ~self.decode_rows(prefill_columns, group)
        return choose_prefill_waves(
            q_lens=self._q_lens, computed=self._computed, rows=rows, group=group, columns=prefill_columns,
            key_tokens=prefill_key_tokens,
            slots_per_head=prefill_resident // num_kv_heads if prefill_resident else 0, wide_built=wide_built,
        )

    def _build_work(
        self, group: int, num_kv_heads: int, resident_waves: int, prefill_columns: int, unit_tokens: int,
        col_tiles: int, prefill_key_tokens: int, prefill_resident: int, prefill_waves: int = 4,
    ) -> DecodeWork:
        computed, q_lens = self._computed, self._q_lens
        batch = self.batch_size
        seq = computed + q_lens
        decode_rows = self.decode_rows(prefill_columns, group)
        nct = -(-(q_lens * group) // 16)
        ngroups = -(-nct // col_tiles)
        pieces = wave_first = jobs = prefill_units = None
        waves = num_jobs = num_partial = num_prefill = per_wave = 0
        blocks = []
        if decode_rows.any():
            max_units = None
            if self.partition_tokens:
                max_units = max(1, self.partition_tokens // unit_tokens)
            piece_tab, first_tab, waves, per_wave, job_tab, num_partial = stream_k_pieces(
                seq=seq, ngroups=ngroups, rows=decode_rows, req_meta=self._req_meta, flat_tables=self._flat,
                num_kv_heads=num_kv_heads,
                resident_waves=resident_waves, block_size=self.block_size, max_units_per_wave=max_units,
                unit_tokens=unit_tokens,
            )
            num_pieces = int(piece_tab.shape[0])
            num_jobs = int(job_tab.shape[0])
            blocks += [piece_tab.reshape(-1), first_tab.reshape(-1)]
            if num_jobs:
                blocks.append(job_tab.reshape(-1))
        prefill_rows = ~decode_rows
        ptab = pjobs = None
        num_pjobs = num_pslots = 0
        if prefill_rows.any():
            ptab, pjobs, num_pslots = prefill_pieces(
                q_lens=q_lens, computed=computed, rows=prefill_rows, req_meta=self._req_meta, group=group,
                columns=prefill_columns, key_tokens=prefill_key_tokens,
                slots_per_head=prefill_resident // num_kv_heads if prefill_resident else 0,
            )
            num_prefill = int(ptab.shape[0])
            num_pjobs = int(pjobs.shape[0])
            blocks.append(ptab.reshape(-1))
            if num_pjobs:
                blocks.append(pjobs.reshape(-1))
        if blocks:
            blob = _stage_int32(np.concatenate(blocks), self.device)
        else:
            blob = None
        off = 0
        if waves:
            pieces = blob[off : off + PIECE_FIELDS * num_pieces].view(num_pieces, PIECE_FIELDS)
            off += PIECE_FIELDS * num_pieces
            wave_first = blob[off : off + waves + 1]
            off += waves + 1
        if num_jobs:
            jobs = blob[off : off + MERGE_FIELDS * num_jobs].view(num_jobs, MERGE_FIELDS)
            off += MERGE_FIELDS * num_jobs
        prefill_jobs = None
        if num_prefill:
            prefill_units = blob[off : off + PREFILL_FIELDS * num_prefill].view(num_prefill, PREFILL_FIELDS)
            off += PREFILL_FIELDS * num_prefill
        if num_pjobs:
            prefill_jobs = blob[off : off + MERGE_FIELDS * num_pjobs].view(num_pjobs, MERGE_FIELDS)
        merge_cols = pmerge_cols = 1
        if num_jobs:
            merge_cols = _job_columns(job_tab, group, 16 * col_tiles)
        if num_pjobs:
            pmerge_cols = _job_columns(pjobs, group, prefill_columns)
        return DecodeWork(pieces, wave_first, waves, jobs, num_jobs, num_partial, per_wave, col_tiles, prefill_units,
                          num_prefill, prefill_jobs, num_pjobs, num_pslots, prefill_waves, merge_cols, pmerge_cols)
