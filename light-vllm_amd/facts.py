"""Array form of one model step's metadata, built by the native host planner.

light-vllm hands the backend Python tuples per step (block tables, computed
counts, query layouts; src/light_vllm/runtime/execution/worker.py:275-285).
``StepFacts`` holds the same facts as flat arrays, produced by one native pass
over the Python objects (``csrc/lvamd_host.cpp``, ``metadata``): the step
plan, the metadata's derived properties and the validation all read them.

``facts_of(metadata)`` accepts this package's ``PagedAttentionMetadata``
(which builds its facts once, on construction) or any object with
light-vllm's metadata attributes (parsed on the call).

The field rules (paged_attention.py:29-62) and block-table rules
(src/light_vllm/runtime/execution/paged_attention.py:110-172) and their
messages are light-vllm's: the native checks report which rule fails first,
in the reference's order, by code; ``FIELD_RULES`` and ``TABLE_RULES`` hold
the messages, raised as ``ValueError`` and the host's ``KVCacheError``.
"""

from __future__ import annotations

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


# Messages of the metadata field rules, by the native planner's rule code
# (paged_attention.py:29-62 holds them in this order).
FIELD_RULES = {
    1: "paged attention metadata must contain at least one request",
    2: "paged attention metadata fields must have the same batch size",
    3: "reserved query counts must have the same batch size",
    4: "readonly prefix counts must have the same batch size",
    5: "computed-token counts must be non-negative integers",
    6: "reserved query counts must cover every actual query",
    7: "readonly prefix counts must be non-negative integers",
    8: "block tables must contain non-negative integers",
    9: "each query parent must be -1 or precede its child",
}

# (name, dtype) of the native planner's buffers, in ``StepFacts.raw`` order.
_ARRAYS = (
    ("flat", np.int32),       # every block table, concatenated
    ("counts", np.int64),     # blocks per table
    ("computed", np.int64),   # num_computed_tokens
    ("reserved", np.int64),   # num_reserved_query_tokens
    ("readonly", np.int64),   # num_readonly_prefix_blocks
    ("q_lens", np.int64),     # queries per request
    ("vis_off", np.int64),    # first ancestor row in ``vis``, -1 for a linear layout
    ("vis_words", np.int64),  # uint32 words per ancestor row
    ("vis", np.uint32),       # ancestor bit rows of the tree layouts
)


def _array_property(index: int, name: str):
    def get(self) -> np.ndarray:
        arrays = self._arrays
        if arrays is None:
            arrays = self._arrays = tuple(np.frombuffer(buf, dtype=dt) for buf, (_, dt) in zip(self.raw, _ARRAYS))
        return arrays[index]

    get.__name__ = name
    return property(get)


class StepFacts:
    """One step's metadata as arrays (one entry per request unless noted).

    ``raw`` holds the native planner's buffers (``_ARRAYS`` order), which the
    planner reads directly; the named numpy views are made on first use.
    """

    __slots__ = ("raw", "batch", "num_tokens", "linear", "_arrays")

    def __init__(self, raw: tuple, num_tokens: int, linear: bool) -> None:
        self.raw = raw
        self.batch = len(raw[1]) // 8
        self.num_tokens = num_tokens  # packed query tokens of the step
        self.linear = linear  # whether every layout is the ordinary causal chain
        self._arrays: tuple[np.ndarray, ...] | None = None

    flat = _array_property(0, "flat")
    counts = _array_property(1, "counts")
    computed = _array_property(2, "computed")
    reserved = _array_property(3, "reserved")
    readonly = _array_property(4, "readonly")
    q_lens = _array_property(5, "q_lens")
    vis_off = _array_property(6, "vis_off")
    vis_words = _array_property(7, "vis_words")
    vis = _array_property(8, "vis")

    @property
    def num_blocks_listed(self) -> int:
        return len(self.raw[0]) // 4

    @property
    def num_vis_words(self) -> int:
        return len(self.raw[8]) // 4

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
        rule, _ = native.host().validate(*self.raw[:5], num_blocks, block_size)
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


def parse_fields(block_tables, computed, layouts, reserved, readonly) -> tuple[tuple, StepFacts]:
    """The metadata constructor's work in one native call: the five fields
    as tuples (defaults filled in) and the step's facts.  The first broken
    field rule, in the reference's order, raises ``ValueError``."""

    found = native.host().metadata(block_tables, computed, layouts, reserved, readonly)
    if type(found) is int:
        raise ValueError(FIELD_RULES[found])
    fields, raw, tokens, linear = found
    return fields, StepFacts(raw, tokens, linear)


def facts_of(metadata) -> StepFacts:
    """The step's facts: kept by this package's metadata, parsed otherwise."""

    found = getattr(metadata, "facts", None)
    if isinstance(found, StepFacts):
        return found
    return parse_fields(metadata.block_tables, metadata.num_computed_tokens, metadata.query_layouts,
                        metadata.num_reserved_query_tokens, metadata.num_readonly_prefix_blocks)[1]
