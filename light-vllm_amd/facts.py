"""Array form of one model step's metadata, built by the native host planner.

light-vllm hands the backend Python tuples per step (block tables, computed
counts, query layouts; src/light_vllm/runtime/execution/worker.py:275-285).
``StepFacts`` holds the same facts as flat arrays, produced by one native pass
over the Python objects (``csrc/lvamd_host.cpp``): the step plan, the
metadata's derived properties and the validation all read these arrays.

``facts_of(metadata)`` accepts this package's ``PagedAttentionMetadata``
(which builds its facts once, on construction) or any object with
light-vllm's metadata attributes (parsed on the call).

The block-table rules and their messages are light-vllm's
(src/light_vllm/runtime/execution/paged_attention.py:110-172): the native
check reports which rule fails first, in the reference's order, and
``raise_table_rule`` raises it with the host's ``KVCacheError``.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from light_vllm_amd import errors, native

# Messages of the block-table rules, by the native planner's rule code.
TABLE_RULES = {
    1: "block table does not cover all scheduled tokens",
    2: "block table contains unused physical blocks",
    3: "block table contains an out-of-range physical block",
    4: "readonly prefix blocks exceed the computed prefix",
    5: "block table aliases a physical block within one request",
    6: "block tables alias a physical block across requests",
}


def _i64(data) -> np.ndarray:
    return np.frombuffer(data, dtype=np.int64)


@dataclass(frozen=True, slots=True, eq=False)
class StepFacts:
    """One step's metadata as arrays (one entry per request unless noted)."""

    flat: np.ndarray       # int32: every block table, concatenated
    counts: np.ndarray     # int64: blocks per table
    computed: np.ndarray   # int64: num_computed_tokens
    reserved: np.ndarray   # int64: num_reserved_query_tokens
    readonly: np.ndarray   # int64: num_readonly_prefix_blocks
    q_lens: np.ndarray     # int64: queries per request
    vis_off: np.ndarray    # int64: first ancestor row in ``vis``, -1 for a linear layout
    vis_words: np.ndarray  # int64: uint32 words per ancestor row
    vis: np.ndarray        # uint32: ancestor bit rows of the tree layouts

    @property
    def batch(self) -> int:
        return int(self.counts.shape[0])

    @property
    def num_tokens(self) -> int:
        return int(self.q_lens.sum())

    @property
    def linear(self) -> bool:
        """Whether every layout is the ordinary causal chain."""

        return bool(np.all(self.vis_off < 0))

    @property
    def table_off(self) -> np.ndarray:
        off = np.zeros(self.batch, dtype=np.int64)
        np.cumsum(self.counts[:-1], out=off[1:])
        return off

    @property
    def q_start(self) -> np.ndarray:
        start = np.zeros(self.batch, dtype=np.int64)
        np.cumsum(self.q_lens[:-1], out=start[1:])
        return start

    def check_coverage(self, block_size: int) -> None:
        """The coverage rule alone (``slot_mapping``'s check): each table has
        exactly ceil((computed + reserved) / block_size) blocks."""

        required = (self.computed + self.reserved + block_size - 1) // block_size
        bad = np.flatnonzero(self.counts != required)
        if bad.size:
            r = int(bad[0])
            raise errors.KVCacheError(TABLE_RULES[1 if self.counts[r] < required[r] else 2])

    def check_tables(self, *, num_blocks: int, block_size: int) -> None:
        """All block-table rules, first failure raised with its message."""

        if num_blocks > np.iinfo(np.int32).max:
            raise ValueError("num_blocks must fit in int32")
        rule, _ = native.host().validate(self.flat, self.counts, self.computed, self.reserved, self.readonly,
                                         num_blocks, block_size)
        if rule:
            raise errors.KVCacheError(TABLE_RULES[rule])

    def slots(self, block_size: int) -> np.ndarray:
        """int64 physical slot of every packed query token."""

        out = np.empty(self.num_tokens, dtype=np.int64)
        meta = np.empty(self.batch * native.REQ_FIELDS, dtype=np.int32)
        if native.host().stage(self.flat, self.counts, self.computed, self.q_lens, self.vis_off, self.vis_words,
                               block_size, out, meta):
            raise errors.KVCacheError(TABLE_RULES[1])
        return out

    def ancestor_rows(self, request: int) -> np.ndarray:
        """bool [q, q] visibility of one request (row i: i and its ancestors)."""

        q = int(self.q_lens[request])
        if self.vis_off[request] < 0:
            return np.tril(np.ones((q, q), dtype=bool))
        words = int(self.vis_words[request])
        off = int(self.vis_off[request])
        rows = self.vis[off : off + q * words].reshape(q, words)
        bits = np.unpackbits(rows.view(np.uint8).reshape(q, words * 4), axis=1, bitorder="little")
        return bits[:, :q].astype(bool)


def parse_ints(values, what: str) -> np.ndarray:
    """int64 array of a sequence of exact non-negative ints; ValueError(what) otherwise."""

    flat, _, status = native.host().flatten((values,), True)
    if status:
        raise ValueError(what)
    return _i64(flat)


def build_facts(block_tables, computed, layouts, reserved, readonly) -> StepFacts:
    """Parse already-checked per-request fields into ``StepFacts``."""

    host = native.host()
    flat, counts, status = host.flatten(block_tables, False)
    if status:
        raise ValueError("block tables must contain non-negative integers")
    q_lens, vis_off, vis_words, vis, bad = host.layouts(layouts)
    if bad:
        raise ValueError("each query parent must be -1 or precede its child")
    return StepFacts(
        flat=np.frombuffer(flat, dtype=np.int32), counts=_i64(counts), computed=computed, reserved=reserved,
        readonly=readonly, q_lens=_i64(q_lens), vis_off=_i64(vis_off), vis_words=_i64(vis_words),
        vis=np.frombuffer(vis, dtype=np.uint32),
    )


def facts_of(metadata) -> StepFacts:
    """The step's facts: kept by this package's metadata, parsed otherwise."""

    found = getattr(metadata, "facts", None)
    if isinstance(found, StepFacts):
        return found
    return build_facts(
        metadata.block_tables,
        parse_ints(metadata.num_computed_tokens, "computed-token counts must be non-negative integers"),
        metadata.query_layouts,
        parse_ints(metadata.num_reserved_query_tokens, "reserved query counts must cover every actual query"),
        parse_ints(metadata.num_readonly_prefix_blocks, "readonly prefix counts must be non-negative integers"),
    )
