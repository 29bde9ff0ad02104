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
* per layer shape: the stream-K split of the decode rows (pieces, each
  wave's first piece, merge jobs) and the prefill units.

Every array comes out of the native host planner (``csrc/lvamd_host.cpp``)
and goes through a pinned staging buffer that is reused step after step
(``Staging``).  The backend asks for every layer shape's work lists before
``commit``, so a step takes one non-blocking H2D copy on the current stream.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
from torch import Tensor

from light_vllm_amd import errors, native
from light_vllm_amd.facts import TABLE_RULES, StepFacts, facts_of

# Requests whose queries x group fit one 16-column MFMA tile use the split-K
# decode kernel; wider ones (prompt chunks, tree verification) use the MFMA
# prefill kernel when it covers the layer's shape, whose waves share each
# K/V tile.
DECODE_MAX_COLUMNS = 16
# Fewest decode tiles per stream-K share: small steps are spread over more
# waves down to this (C1, 4 sequences of 38-512 tokens in fp32: 10.6-10.8 us
# per step at one tile per share against 11.5 at two, once the host path no
# longer set the step's pace); steps that fill the resident waves are not
# affected.
DECODE_MIN_UNITS_PER_WAVE = 1
# Smallest key range (in prefill key tiles) the planner gives one prefill
# workgroup when it splits units to fill the GPU.
PREFILL_MIN_TILES = 4
# Compute units of an MI355X; the planner aims for several waves per CU.
NUM_CUS = 256

PIECE_FIELDS = native.PIECE_FIELDS
PREFILL_FIELDS = native.PREFILL_FIELDS
MERGE_FIELDS = native.MERGE_FIELDS
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
PREFILL_WIDE_MAX_TILES = 20  # mean key tiles per unit up to which 8-wave prefill workgroups win

_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream(device: torch.device) -> int:
    """The current HIP stream of ``device`` as a raw handle (torch's own
    accessor when present: it skips building a Stream object per call)."""

    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


class Staging:
    """Pinned host buffers for per-step uploads, reused round-robin.

    A buffer is refilled only after the H2D copy that last read it has
    finished (an event per buffer, as light-vllm's single-step staging
    buffer waits for the previous copy, cuda_staging.py:27-49); with several
    buffers in the ring that wait is normally already over.  On a CPU device
    the arrays are handed over as CPU tensors (the planner's tests).
    """

    DEPTH = 4
    MIN_ENTRIES = 1 << 16  # int32 entries of a fresh buffer (256 KiB)

    def __init__(self, device: torch.device) -> None:
        self.device = torch.device(device)
        self._gpu = self.device.type == "cuda"
        self._lib = native.load() if self._gpu else None
        self._host: list[Tensor | None] = [None] * self.DEPTH
        self._views: list[np.ndarray | None] = [None] * self.DEPTH
        self._events: list[object | None] = [None] * self.DEPTH
        self._next = 0
        self._slot = -1

    def take(self, n: int = 0) -> np.ndarray:
        """The next buffer of the ring, whole (at least ``n`` int32 entries),
        once the copy that last read it has finished."""

        if not self._gpu:
            return np.zeros(max(n, self.MIN_ENTRIES), dtype=np.int32)
        slot = self._next
        self._next = (slot + 1) % self.DEPTH
        event = self._events[slot]
        if event is not None:
            event.synchronize()
        self._slot = slot
        view = self._views[slot]
        if view is None or view.shape[0] < n:
            view = self.grow(n)
        return view

    def grow(self, n: int) -> np.ndarray:
        """Replace the buffer ``take`` returned by one of at least ``n`` entries."""

        if not self._gpu:
            return np.zeros(max(n, self.MIN_ENTRIES), dtype=np.int32)
        slot = self._slot
        old = self._host[slot]
        size = max(n, self.MIN_ENTRIES, 2 * old.numel() if old is not None else 0)
        host = self._host[slot] = torch.empty(size, dtype=torch.int32, pin_memory=True)
        view = self._views[slot] = host.numpy()
        return view

    def buffer(self, n: int) -> np.ndarray:
        """A writable int32 host array of ``n`` entries for the next upload."""

        return self.take(n)[:n]

    def upload(self, array: np.ndarray) -> Tensor:
        """The device copy of a prefix of the buffer ``take`` returned
        (non-blocking, on the current stream)."""

        if not self._gpu:
            return torch.from_numpy(array)
        slot = self._slot
        n = array.shape[0]
        dev = torch.empty(n, dtype=torch.int32, device=self.device)
        event = self._events[slot]
        if event is None:
            event = self._events[slot] = torch.cuda.Event()
            event.record()  # creates the HIP event behind it
        # One library call: the async H2D copy, then the slot's event.
        native.check(self._lib.lvamd_stage_upload(dev.data_ptr(), self._host[slot].data_ptr(), 4 * n,
                                                  event.cuda_event, current_stream(self.device)),
                     "lvamd_stage_upload")
        return dev

    def stage(self, parts: list[np.ndarray]) -> tuple[Tensor, list[int]]:
        """Upload ``parts`` (int32 arrays) in one copy: the device tensor and
        each part's offset in it (int32 entries)."""

        sizes = [p.size for p in parts]
        buf = self.buffer(int(sum(sizes)))
        offsets, off = [], 0
        for p, n in zip(parts, sizes):
            buf[off : off + n] = p.reshape(-1)
            offsets.append(off)
            off += n
        return self.upload(buf[:off]), offsets


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


class DecodeWork:
    """Work lists of one layer shape: host arrays (int32) and, once the plan
    is uploaded, the device address of each.  The tensor properties give the
    host arrays as CPU tensors (inspection and tests)."""

    __slots__ = ("pieces_host", "wave_first_host", "jobs_host", "units_host", "prefill_jobs_host",
                 "waves_per_head", "num_jobs", "num_partial_slots", "units_per_wave", "col_tiles", "group_waves",
                 "num_prefill_units", "num_prefill_jobs", "num_prefill_partial_slots", "prefill_waves",
                 "merge_columns", "prefill_merge_columns", "pieces_ptr", "wave_first_ptr", "jobs_ptr",
                 "units_ptr", "prefill_jobs_ptr", "_staged")

    def __init__(self, *, col_tiles: int, prefill_waves: int) -> None:
        self.col_tiles = col_tiles  # column tiles per decode wave (partials hold 16 * col_tiles columns)
        # Decode waves per workgroup: 1 (stream-K shares, merge launch) or 4
        # (workgroup split: one segment per workgroup, merged in LDS).
        self.group_waves = 1
        self.prefill_waves = prefill_waves  # prefill workgroup shape: 4 waves x 2 column tiles or 8 x 1
        self.pieces_host = self.wave_first_host = self.jobs_host = None
        self.units_host = self.prefill_jobs_host = None
        self.waves_per_head = self.num_jobs = self.num_partial_slots = self.units_per_wave = 0
        self.num_prefill_units = self.num_prefill_jobs = self.num_prefill_partial_slots = 0
        self.merge_columns = self.prefill_merge_columns = 1  # most columns any merge job has
        self.pieces_ptr = self.wave_first_ptr = self.jobs_ptr = self.units_ptr = self.prefill_jobs_ptr = None
        self._staged = None  # (uploaded blob, {list name: (offset, rows, fields)}) of a fused plan

    @classmethod
    def staged(cls, row: tuple[int, ...], blob: Tensor) -> "DecodeWork":
        """A layer shape's work as ``plan_step`` placed it in ``blob`` (the
        uploaded step buffer): counts from ``row``, lists only on the device."""

        (ctw, waves, wph, per_wave, slots, njobs, mcols, nunits, npjobs, pslots, pmcols,
         o_pieces, o_first, o_jobs, o_units, o_pjobs, npieces, group_waves) = row
        work = cls(col_tiles=ctw, prefill_waves=waves)
        work.group_waves = group_waves
        work.waves_per_head, work.units_per_wave, work.num_partial_slots = wph, per_wave, slots
        work.num_jobs, work.merge_columns = njobs, mcols
        work.num_prefill_units, work.num_prefill_jobs = nunits, npjobs
        work.num_prefill_partial_slots, work.prefill_merge_columns = pslots, pmcols
        base = blob.data_ptr()
        if o_pieces >= 0:
            work.pieces_ptr, work.wave_first_ptr = base + 4 * o_pieces, base + 4 * o_first
        if o_jobs >= 0:
            work.jobs_ptr = base + 4 * o_jobs
        if o_units >= 0:
            work.units_ptr = base + 4 * o_units
        if o_pjobs >= 0:
            work.prefill_jobs_ptr = base + 4 * o_pjobs
        work._staged = (blob, {
            "pieces": (o_pieces, npieces, PIECE_FIELDS), "wave_first": (o_first, wph + 1, 1),
            "jobs": (o_jobs, njobs, MERGE_FIELDS), "prefill_units": (o_units, nunits, PREFILL_FIELDS),
            "prefill_jobs": (o_pjobs, npjobs, MERGE_FIELDS),
        })
        return work

    def parts(self) -> list[tuple[str, np.ndarray]]:
        """(pointer attribute, array) of every list to upload."""

        found = [("pieces_ptr", self.pieces_host), ("wave_first_ptr", self.wave_first_host),
                 ("jobs_ptr", self.jobs_host), ("units_ptr", self.units_host),
                 ("prefill_jobs_ptr", self.prefill_jobs_host)]
        return [(name, array) for name, array in found if array is not None and array.size]

    def _tensor(self, array, name: str):
        if self._staged is None:
            return None if array is None or not array.size else torch.from_numpy(array)
        blob, lists = self._staged
        off, rows, fields = lists[name]
        if off < 0 or not rows:
            return None
        flat = blob[off : off + rows * fields].cpu()
        return flat if fields == 1 else flat.view(rows, fields)

    @property
    def pieces(self) -> Tensor | None:  # int32 [n_pieces, 16]
        return self._tensor(self.pieces_host, "pieces")

    @property
    def wave_first(self) -> Tensor | None:  # int32 [waves_per_head + 1]
        return self._tensor(self.wave_first_host, "wave_first")

    @property
    def jobs(self) -> Tensor | None:  # int32 [n_jobs, 8]
        return self._tensor(self.jobs_host, "jobs")

    @property
    def prefill_units(self) -> Tensor | None:  # int32 [n_prefill_units, 8]
        return self._tensor(self.units_host, "prefill_units")

    @property
    def prefill_jobs(self) -> Tensor | None:  # int32 [n, 8] merge jobs of split prefill units
        return self._tensor(self.prefill_jobs_host, "prefill_jobs")


def _as_i32(data) -> np.ndarray:
    return np.frombuffer(data, dtype=np.int32)


class StepPlan:
    """Device-resident metadata of one model step (valid for all of its layers).

    The step facts, and the work lists of any layer shape asked for before
    ``commit``, share one upload; a shape asked for later is uploaded on its
    own.  Kernels take the ``*_ptr`` device addresses; the tensor properties
    (``slots``, ``req_meta``, ``tables``, ``vis``) are views for inspection.
    """

    def __init__(
        self,
        metadata,
        *,
        block_size: int,
        device: torch.device,
        partition_tokens: int | None = None,
        num_blocks: int | None = None,
        staging: Staging | None = None,
        defer_upload: bool = False,
        shapes: "LayerShapes | None" = None,
    ) -> None:
        """With ``num_blocks`` the block tables are validated first, with the
        rules and messages of ``PagedAttentionMetadata.validate_block_tables``
        (paged_attention.py:138-173), in the native planner.  With
        ``defer_upload`` nothing is copied until ``commit()``.

        With ``shapes`` (and ``num_blocks``) the whole step is planned in one
        native call (``plan_step``): validation, the step facts and every
        listed layer shape's work lists, written straight into a pinned
        staging buffer and uploaded at once; the plan is committed."""

        self.block_size = block_size
        self.device = torch.device(device)
        self.partition_tokens = partition_tokens
        self._staging = staging if staging is not None else Staging(self.device)
        facts: StepFacts = facts_of(metadata)
        self.facts = facts
        self.num_tokens = tokens = facts.num_tokens
        self.batch_size = batch = facts.batch
        self.has_tree = not facts.linear
        self._work: dict[tuple[int, ...], DecodeWork] = {}
        self._col_tiles: dict[tuple[int, int, int], int] = {}
        self._pending: list[DecodeWork] = []
        self._late_blobs: list[Tensor] = []  # uploads of work lists asked for after commit
        self._blob: Tensor | None = None
        self._committed = False
        self._req_meta_host: np.ndarray | None = None
        # Bound launch arguments per layer shape, filled by the backend.
        self.launches: dict[tuple, object] = {}
        # (start, length) in int32 entries of slots, req_meta, tables and vis in the upload.
        self._spans: tuple[tuple[int, int], ...] = ()
        nflat, nvis = facts.num_blocks_listed, facts.num_vis_words
        if shapes is not None:
            if num_blocks is None:
                raise ValueError("a step planned with layer shapes validates its tables: pass num_blocks")
            self._plan_step(num_blocks, shapes, (2 * tokens, batch * native.REQ_FIELDS, nflat, nvis))
            return
        if num_blocks is not None:
            facts.check_tables(num_blocks=num_blocks, block_size=block_size)
        # Step facts as one int32 array: [slots as int32 pairs | req_meta | tables | vis].
        sizes = (2 * tokens, batch * native.REQ_FIELDS, max(nflat, 1), max(nvis, 1))
        offs = np.concatenate(([0], np.cumsum(sizes))).tolist()
        self._spans = tuple((offs[i], sizes[i]) for i in range(4))
        arr = np.zeros(offs[-1], dtype=np.int32)
        req_meta = arr[offs[1] : offs[2]]
        if native.host().stage(facts.flat, facts.counts, facts.computed, facts.q_lens, facts.vis_off,
                               facts.vis_words, block_size, arr[offs[0] : offs[1]].view(np.int64), req_meta):
            facts.check_coverage(block_size)
            raise ValueError("a query position lies past its block table")
        arr[offs[2] : offs[2] + nflat] = facts.flat
        arr[offs[3] : offs[3] + nvis] = facts.vis.view(np.int32)
        self._req_meta_host = req_meta
        self._facts_host = arr
        if not defer_upload:
            self.commit()

    def _plan_step(self, num_blocks: int, shapes: "LayerShapes", sizes: tuple[int, int, int, int]) -> None:
        raw = self.facts.raw
        host = native.host()
        staging = self._staging
        buf = staging.take()
        while True:
            found = host.plan_step(*raw, num_blocks, self.block_size, shapes.array, COL_TILES4_COST,
                                   float(PREFILL_WIDE_MAX_TILES), buf)
            if type(found) is int:
                raise errors.KVCacheError(TABLE_RULES[found])
            used, offs, rows = found
            if offs is not None:
                break
            buf = staging.grow(used)
        blob = self._blob = staging.upload(buf[:used])
        base = blob.data_ptr()
        self._spans = tuple(zip(offs, sizes))
        self.slots_ptr, self.req_meta_ptr, self.tables_ptr, self.vis_ptr = (base + 4 * o for o in offs)
        for key, row in zip(shapes.keys, rows):
            self._work[key] = DecodeWork.staged(row, blob)
        self._committed = True

    @property
    def _req_meta(self) -> np.ndarray:
        """int32 [B * 8] per-request records on the host (built on first use
        when the step was planned in one call)."""

        if self._req_meta_host is None:
            f = self.facts
            meta = np.empty(self.batch_size * native.REQ_FIELDS, dtype=np.int32)
            slots = np.empty(self.num_tokens, dtype=np.int64)
            native.host().stage(f.flat, f.counts, f.computed, f.q_lens, f.vis_off, f.vis_words, self.block_size,
                                slots, meta)
            self._req_meta_host = meta
        return self._req_meta_host

    def commit(self) -> None:
        """Upload the step facts and every work list built so far (one copy)."""

        if self._committed:
            return
        parts = [self._facts_host]
        owners: list[tuple[DecodeWork | None, str]] = [(None, "")]
        for work in self._pending:
            for name, array in work.parts():
                parts.append(array)
                owners.append((work, name))
        blob, offsets = self._staging.stage(parts)
        base = blob.data_ptr()
        for (work, name), off in zip(owners, offsets):
            if work is not None:
                setattr(work, name, base + 4 * off)
        self._blob = blob
        spans = self._spans
        self.slots_ptr = base + 4 * spans[0][0]
        self.req_meta_ptr = base + 4 * spans[1][0]
        self.tables_ptr = base + 4 * spans[2][0]
        self.vis_ptr = base + 4 * spans[3][0]
        self._pending = []
        self._committed = True

    def _view(self, i: int) -> Tensor:
        self.commit()
        start, length = self._spans[i]
        return self._blob[start : start + length]

    @property
    def slots(self) -> Tensor:  # int64 [T]
        return self._view(0).view(torch.int64)

    @property
    def req_meta(self) -> Tensor:  # int32 [B * 8]
        return self._view(1)

    @property
    def tables(self) -> Tensor:  # int32 flat block tables
        return self._view(2)

    @property
    def vis(self) -> Tensor:  # uint32 ancestor rows, as int32
        return self._view(3)

    @property
    def num_query_tokens(self) -> int:
        return self.num_tokens

    # -- work lists ---------------------------------------------------------
    def decode_rows(self, prefill_columns: int, group: int = 1) -> np.ndarray:
        """Requests the decode kernel serves (all of them without a prefill kernel)."""

        if prefill_columns > 0:
            return self.facts.q_lens * group <= DECODE_MAX_COLUMNS
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
            rows = self.decode_rows(prefill_columns, group)
            q_lens = self.facts.q_lens[rows]
            seq = self.facts.computed[rows] + q_lens
            nct = -(-(q_lens * group) // 16)
            one = float((seq * nct).sum())
            four = float((seq * -(-nct // 4)).sum()) * COL_TILES4_COST
            found = self._col_tiles[key] = 4 if four < one else 1
        return found

    def prefill_waves(self, group: int, num_kv_heads: int, prefill_columns: int, prefill_key_tokens: int,
                      prefill_resident: int, wide_built: bool) -> int:
        """The prefill workgroup shape (4 or 8 waves) for this step's wide rows."""

        rows = ~self.decode_rows(prefill_columns, group)
        return choose_prefill_waves(
            q_lens=self.facts.q_lens, computed=self.facts.computed, rows=rows, group=group, columns=prefill_columns,
            key_tokens=prefill_key_tokens,
            slots_per_head=prefill_resident // num_kv_heads if prefill_resident else 0, wide_built=wide_built,
        )

    def work(
        self, group: int, num_kv_heads: int, resident_waves: int = 8 * NUM_CUS, prefill_columns: int = 0,
        unit_tokens: int = UNIT_TOKENS, col_tiles: int = 1, prefill_key_tokens: int = 64,
        prefill_resident: int = 0, prefill_waves: int = 4, shared_prefix: bool = False, xcds: int = 0,
        prefill_order: int = 0, split_groups: int = 0, split_waves: int = 8,
    ) -> DecodeWork:
        """Work lists for layers of this (group, kv heads) shape.

        ``resident_waves`` is how many decode waves the GPU holds at once,
        ``prefill_columns`` the prefill kernel's unit width (0: every request
        goes through the decode kernel), ``unit_tokens`` the decode kernel's
        tile and ``col_tiles`` its column tiles per wave; ``prefill_key_tokens``
        is the prefill kernel's key tile and ``prefill_resident`` how many
        prefill workgroups of shape ``prefill_waves`` the GPU holds (0: never
        split prefill units); ``shared_prefix`` attends prefixes that runs of
        prefill requests share once per span (the backend's default);
        ``xcds`` > 1 orders the prefill units per XCD of a device with that
        many (the backend passes the device's count): ``prefill_order`` 0
        keeps each request's units on one XCD when the simulated packing is
        no slower, 1 always, 2 never; ``split_groups`` > 0 (the resident
        workgroups of the workgroup-split decode kernel) lets the planner
        give each segment a workgroup of ``split_waves`` waves when that is
        no slower than stream-K with its merge launch.  The library reports the kernel
        figures per dtype and head size.
        """

        key = (group, num_kv_heads, resident_waves, prefill_columns, unit_tokens, col_tiles, prefill_key_tokens,
               prefill_resident, prefill_waves, bool(shared_prefix), int(xcds), int(prefill_order), int(split_groups),
               int(split_waves))
        found = self._work.get(key)
        if found is None:
            found = self._build_work(*key)
            self._register(key, found)
        return found

    def layer_work(self, kernel_facts: tuple[int, ...]) -> DecodeWork:
        """Work lists of one layer shape from the library's kernel facts
        (``KERNEL_FACTS`` order): one native call chooses this step's column
        tiles per decode wave and prefill workgroup shape, then builds both
        lists.  Cached per facts tuple; uploaded with the step when asked for
        before ``commit``."""

        found = self._work.get(kernel_facts)
        if found is None:
            ctw, waves, dec, pre = native.host().layer_work(
                self._req_meta, self.facts.raw[0], np.asarray(kernel_facts, dtype=np.int64), COL_TILES4_COST,
                float(PREFILL_WIDE_MAX_TILES),
            )
            found = DecodeWork(col_tiles=int(ctw), prefill_waves=int(waves))
            _fill_work(found, dec, pre)
            self._register(kernel_facts, found)
        return found

    def _register(self, key: tuple, work: DecodeWork) -> None:
        self._work[key] = work
        if not self._committed:
            self._pending.append(work)
            return
        parts = work.parts()
        if parts:
            blob, offsets = self._staging.stage([array for _, array in parts])
            for (name, _), off in zip(parts, offsets):
                setattr(work, name, blob.data_ptr() + 4 * off)
            self._late_blobs.append(blob)

    def _build_work(
        self, group: int, num_kv_heads: int, resident_waves: int, prefill_columns: int, unit_tokens: int,
        col_tiles: int, prefill_key_tokens: int, prefill_resident: int, prefill_waves: int, shared_prefix: bool,
        xcds: int, prefill_order: int, split_groups: int, split_waves: int,
    ) -> DecodeWork:
        host = native.host()
        work = DecodeWork(col_tiles=col_tiles, prefill_waves=prefill_waves)
        max_cols = DECODE_MAX_COLUMNS if prefill_columns > 0 else 0
        q_cols = self.facts.q_lens * group
        dec = pre = None
        if max_cols == 0 or bool(np.any(q_cols <= max_cols)):
            max_units = max(1, self.partition_tokens // unit_tokens) if self.partition_tokens else 0
            dec = host.decode_work(self._req_meta, self.facts.flat, group, col_tiles, max_cols, num_kv_heads,
                                   resident_waves, self.block_size, DECODE_MIN_UNITS_PER_WAVE, max_units,
                                   unit_tokens, split_groups,
                                   split_waves)
        if max_cols and bool(np.any(q_cols > max_cols)):
            slots_per_head = prefill_resident // num_kv_heads if prefill_resident else 0
            pre = host.prefill_work(self._req_meta, self.facts.raw[0], group, prefill_columns, prefill_key_tokens,
                                    slots_per_head, PREFILL_MIN_TILES, max_cols, self.block_size,
                                    int(shared_prefix), num_kv_heads, xcds, prefill_order)
        _fill_work(work, dec, pre)
        return work


# Order of the kernel facts ``StepPlan.layer_work`` takes (one int each).
KERNEL_FACTS = (
    "group", "num_kv_heads", "block_size", "prefill_columns", "prefill_key_tokens", "split_prefill",
    "forced_col_tiles", "forced_prefill_waves", "max_col_tiles", "wide_prefill_built",
    "resident_waves_1", "tile_tokens_1", "resident_waves_4", "tile_tokens_4",
    "prefill_resident_4", "prefill_resident_8", "partition_tokens", "decode_max_columns",
    "min_units_per_wave", "prefill_min_tiles", "shared_prefix", "xcds", "prefill_order", "split_groups",
    "split_waves",
)


class LayerShapes:
    """The kernel-facts rows (``KERNEL_FACTS`` order) of every layer shape a
    step plans for: the rows as tuples (keys of the plan's work lists) and as
    one int64 array (the native planner's argument)."""

    __slots__ = ("keys", "array")

    def __init__(self, rows) -> None:
        self.keys = tuple(tuple(int(v) for v in row) for row in rows)
        if any(len(row) != len(KERNEL_FACTS) for row in self.keys):
            raise ValueError(f"each layer shape needs {len(KERNEL_FACTS)} kernel facts")
        self.array = np.asarray(self.keys, dtype=np.int64).reshape(-1)


def _fill_work(work: DecodeWork, dec, pre) -> None:
    """Store the native planner's decode and prefill results in ``work``."""

    if dec is not None:
        pieces, first, jobs, waves, per_wave, slots, merge_cols, group_waves = dec
        work.group_waves = int(group_waves)
        work.pieces_host = _as_i32(pieces).reshape(-1, PIECE_FIELDS)
        work.wave_first_host = _as_i32(first)
        work.jobs_host = _as_i32(jobs).reshape(-1, MERGE_FIELDS)
        work.waves_per_head, work.units_per_wave = int(waves), int(per_wave)
        work.num_partial_slots, work.num_jobs = int(slots), int(work.jobs_host.shape[0])
        work.merge_columns = int(merge_cols)
    if pre is not None:
        units, jobs, pslots, _, merge_cols = pre
        work.units_host = _as_i32(units).reshape(-1, PREFILL_FIELDS)
        work.prefill_jobs_host = _as_i32(jobs).reshape(-1, MERGE_FIELDS)
        work.num_prefill_units = int(work.units_host.shape[0])
        work.num_prefill_jobs = int(work.prefill_jobs_host.shape[0])
        work.num_prefill_partial_slots = int(pslots)
        work.prefill_merge_columns = int(merge_cols)
