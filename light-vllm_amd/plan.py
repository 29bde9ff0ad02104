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
* per (group size, kv heads): split-K work units and merge jobs for requests
  on the decode path, and query blocks for requests on the prefill path.

All int32 facts of a step share one pinned buffer and one non-blocking H2D
copy on the current stream; the work lists of each group size add one more.
"""

from __future__ import annotations

import itertools
from dataclasses import dataclass

import numpy as np
import torch
from torch import Tensor

from light_vllm_amd.layout import is_linear, query_visibility

# Requests with at most this many queries use the split-K decode kernel;
# longer runs use the MFMA prefill kernel.
DECODE_MAX_QUERIES = 16
# Query tokens per prefill work unit.
PREFILL_QUERY_BLOCK = 64
# Compute units of an MI355X; the planner aims for several waves per CU.
NUM_CUS = 256

_BIT_WEIGHTS = (np.uint64(1) << np.arange(32, dtype=np.uint64)).astype(np.uint64)


def _stage_int32(array: np.ndarray, device: torch.device) -> Tensor:
    """One pinned host buffer, one non-blocking copy on the current stream."""

    host = torch.from_numpy(np.ascontiguousarray(array, dtype=np.int32))
    if device.type == "cuda":
        host = host.pin_memory()
    return host.to(device, non_blocking=True)


@dataclass(frozen=True, slots=True)
class DecodeWork:
    units: Tensor | None  # int32 [n_units, 4]
    num_units: int
    jobs: Tensor | None  # int32 [n_jobs, 4]
    num_jobs: int
    num_partial_slots: int
    partition_tokens: int
    prefill_units: Tensor | None  # int32 [n_prefill_units, 4]
    num_prefill_units: int


class StepPlan:
    """Device-resident metadata of one model step (valid for all of its layers)."""

    def __init__(self, metadata, *, block_size: int, device: torch.device, use_prefill: bool = True) -> None:
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
        self.use_prefill = use_prefill

        self._computed = computed
        self._q_lens = q_lens
        self._work: dict[tuple[int, int], DecodeWork] = {}

    # -- work lists ---------------------------------------------------------
    def work(self, group: int, num_kv_heads: int) -> DecodeWork:
        key = (group, num_kv_heads)
        found = self._work.get(key)
        if found is None:
            found = self._build_work(group, num_kv_heads)
            self._work[key] = found
        return found

    def _choose_partition(self, seq: np.ndarray, decode_rows: np.ndarray, nct: np.ndarray, num_kv_heads: int) -> int:
        """Partition length (tokens): long enough to amortise the merge, short
        enough that the decode grid fills every CU several times."""

        for tokens in (512, 256, 128, 64, 32):
            waves = int((np.ceil(seq[decode_rows] / tokens) * nct[decode_rows]).sum()) * num_kv_heads
            if waves >= 8 * NUM_CUS:
                return tokens
        return 32

    def _build_work(self, group: int, num_kv_heads: int) -> DecodeWork:
        computed, q_lens = self._computed, self._q_lens
        batch = self.batch_size
        seq = computed + q_lens
        if self.use_prefill:
            decode_rows = q_lens <= DECODE_MAX_QUERIES
        else:
            decode_rows = np.ones(batch, dtype=bool)
        nct = -(-(q_lens * group) // 16)
        units = jobs = prefill_units = None
        num_units = num_jobs = num_partial = num_prefill = 0
        part_tokens = 256
        if decode_rows.any():
            part_tokens = self._choose_partition(seq, decode_rows, nct, num_kv_heads)
            nparts = np.where(decode_rows, -(-seq // part_tokens), 0)
            per_req = nparts * np.where(decode_rows, nct, 0)
            num_units = int(per_req.sum())
            req = np.repeat(np.arange(batch), per_req)
            starts = np.zeros(batch, dtype=np.int64)
            np.cumsum(per_req[:-1], out=starts[1:])
            local = np.arange(num_units) - starts[req]
            part = local % nparts[req]
            ctile = local // nparts[req]
            multi = nparts[req] > 1
            pslot = np.where(multi, np.cumsum(multi) - 1, -1)
            num_partial = int(multi.sum())
            table = np.stack([req, part, ctile, pslot], axis=1)
            first = multi & (part == 0)
            job_tab = np.stack([req[first], ctile[first], pslot[first], nparts[req[first]]], axis=1)
            num_jobs = int(job_tab.shape[0])
            blocks = [table.reshape(-1)]
            if num_jobs:
                blocks.append(job_tab.reshape(-1))
        else:
            blocks = []
        prefill_rows = ~decode_rows
        if prefill_rows.any():
            nblk = np.where(prefill_rows, -(-q_lens // PREFILL_QUERY_BLOCK), 0)
            num_prefill = int(nblk.sum())
            req = np.repeat(np.arange(batch), nblk)
            starts = np.zeros(batch, dtype=np.int64)
            np.cumsum(nblk[:-1], out=starts[1:])
            qb = (np.arange(num_prefill) - starts[req]) * PREFILL_QUERY_BLOCK
            nq = np.minimum(PREFILL_QUERY_BLOCK, q_lens[req] - qb)
            # Heaviest blocks (most visible keys) first: better tail balance.
            work = computed[req] + qb + nq
            order = np.argsort(-work, kind="stable")
            ptab = np.stack([req[order], qb[order], nq[order], np.zeros(num_prefill, dtype=np.int64)], axis=1)
            blocks.append(ptab.reshape(-1))
        if blocks:
            blob = _stage_int32(np.concatenate(blocks), self.device)
        else:
            blob = None
        off = 0
        if num_units:
            units = blob[off : off + 4 * num_units].view(num_units, 4)
            off += 4 * num_units
        if num_jobs:
            jobs = blob[off : off + 4 * num_jobs].view(num_jobs, 4)
            off += 4 * num_jobs
        if num_prefill:
            prefill_units = blob[off : off + 4 * num_prefill].view(num_prefill, 4)
        return DecodeWork(units, num_units, jobs, num_jobs, num_partial, part_tokens, prefill_units, num_prefill)
