"""Per-step batch facts of a packed paged-attention batch.

The contract is light-vllm's ``PagedAttentionMetadata``
(src/light_vllm/runtime/execution/paged_attention.py:18-206): the same
fields and defaults, the same derived properties and methods, the same
validation messages, and the same rule firing first when several are broken.
The backend reads a metadata object only through these attributes, so
light-vllm's own class can be passed in its place.

How it is built here: construction checks the batch shape, then hands every
integer field to the native host planner in one pass each (exact-int and
sign checks in C), and keeps the result as ``facts`` (``StepFacts``: flat
int32 block ids, per-request arrays, packed ancestor rows).  The derived
properties, ``slot_mapping``, ``validate_block_tables`` and the backend's
step plan all read those arrays, so a step's tuples are walked once.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable

import numpy as np
import torch
from torch import Tensor

from light_vllm_amd.facts import StepFacts, build_facts, parse_ints
from light_vllm_amd.interfaces import QueryLayout


def _first_failure(rules: tuple[tuple[Callable[[], bool], str], ...]) -> None:
    for holds, message in rules:
        if not holds():
            raise ValueError(message)


@dataclass(frozen=True, slots=True)
class PagedAttentionMetadata:
    """Block tables, computed-token counts and query layouts of one step."""

    block_tables: tuple[tuple[int, ...], ...]
    num_computed_tokens: tuple[int, ...]
    query_layouts: tuple[QueryLayout, ...]
    # Actual queries plus the scheduler's reserved, possibly unused, slots.
    num_reserved_query_tokens: tuple[int, ...] = ()
    num_readonly_prefix_blocks: tuple[int, ...] = ()
    facts: StepFacts = field(init=False, repr=False, compare=False)

    def __post_init__(self) -> None:
        tables = tuple(map(tuple, self.block_tables))
        computed = tuple(self.num_computed_tokens)
        layouts = tuple(self.query_layouts)
        batch = len(tables)
        _first_failure((
            (lambda: batch > 0, "paged attention metadata must contain at least one request"),
            (lambda: len(computed) == batch == len(layouts),
             "paged attention metadata fields must have the same batch size"),
        ))
        # Empty reserved / readonly fields default per request: the layout's
        # query count, and no readonly prefix.
        reserved = tuple(self.num_reserved_query_tokens) or tuple(len(layout) for layout in layouts)
        readonly = tuple(self.num_readonly_prefix_blocks) or (0,) * batch
        _first_failure((
            (lambda: len(reserved) == batch, "reserved query counts must have the same batch size"),
            (lambda: len(readonly) == batch, "readonly prefix counts must have the same batch size"),
        ))
        computed_arr = parse_ints(computed, "computed-token counts must be non-negative integers")
        q_lens = np.fromiter(map(len, layouts), dtype=np.int64, count=batch)
        reserved_arr = parse_ints(reserved, "reserved query counts must cover every actual query")
        if np.any(reserved_arr < q_lens):
            raise ValueError("reserved query counts must cover every actual query")
        readonly_arr = parse_ints(readonly, "readonly prefix counts must be non-negative integers")
        facts = build_facts(tables, computed_arr, layouts, reserved_arr, readonly_arr)
        object.__setattr__(self, "block_tables", tables)
        object.__setattr__(self, "num_computed_tokens", computed)
        object.__setattr__(self, "query_layouts", layouts)
        object.__setattr__(self, "num_reserved_query_tokens", reserved)
        object.__setattr__(self, "num_readonly_prefix_blocks", readonly)
        object.__setattr__(self, "facts", facts)

    @property
    def batch_size(self) -> int:
        return self.facts.batch

    @property
    def query_lengths(self) -> tuple[int, ...]:
        return tuple(self.facts.q_lens.tolist())

    @property
    def query_start_loc(self) -> tuple[int, ...]:
        return (0, *np.cumsum(self.facts.q_lens).tolist())

    @property
    def num_query_tokens(self) -> int:
        return self.facts.num_tokens

    @property
    def has_only_linear_queries(self) -> bool:
        return self.facts.linear

    @property
    def request_indices(self) -> tuple[int, ...]:
        return tuple(np.repeat(np.arange(self.facts.batch), self.facts.q_lens).tolist())

    def slot_mapping(self, *, block_size: int, device: torch.device) -> Tensor:
        """Physical slot of every packed query token: table[p // bs] * bs + p % bs
        for p = computed + query offset; each table must cover exactly the
        computed and reserved tokens."""

        self.facts.check_coverage(block_size)
        return torch.from_numpy(self.facts.slots(block_size)).to(device)

    def validate_block_tables(self, *, num_blocks: int, block_size: int) -> None:
        """Prove the tables safe to read and write this step: exact coverage,
        ids in range, readonly prefix within the computed tokens, no id twice
        in a table, and an id shared by several tables only at the same
        logical index inside every sharer's readonly prefix."""

        self.facts.check_tables(num_blocks=num_blocks, block_size=block_size)

    def visibility_tensor(self, *, device: torch.device) -> tuple[Tensor, Tensor]:
        """Row-major q x q ancestor masks of all requests, concatenated, and their int32 starts."""

        masks = [self.facts.ancestor_rows(r).reshape(-1) for r in range(self.facts.batch)]
        starts = np.zeros(self.facts.batch + 1, dtype=np.int32)
        np.cumsum(self.facts.q_lens ** 2, out=starts[1:])
        return (
            torch.from_numpy(np.concatenate(masks)).to(device),
            torch.from_numpy(starts).to(device),
        )

    def request_indices_tensor(self, *, device: torch.device) -> Tensor:
        idx = np.repeat(np.arange(self.facts.batch, dtype=np.int32), self.facts.q_lens)
        return torch.from_numpy(idx).to(device)

    def visible_logical_positions(self, row: int) -> tuple[tuple[int, ...], ...]:
        """Logical key positions every query of request ``row`` may read:
        the computed prefix, then the visible queries of this step."""

        computed = int(self.facts.computed[row])
        rows = self.facts.ancestor_rows(row)
        return tuple(
            tuple(range(computed)) + tuple((computed + np.flatnonzero(visible)).tolist())
            for visible in rows
        )
