"""Per-step batch facts of a packed paged-attention batch.

The contract is light-vllm's ``PagedAttentionMetadata``
(src/light_vllm/runtime/execution/paged_attention.py:18-206): the same
fields and defaults, the same derived properties and methods, the same
validation messages, and the same rule firing first when several are broken.
The backend reads a metadata object only through these attributes, so
light-vllm's own class can be passed in its place.

How it is built here: construction hands the five fields to the native host
planner in one call, which applies the field rules (exact-int, sign, batch
and coverage checks in C, first failure by the reference's order) and
returns the normalized tuples and ``facts`` (``StepFacts``: flat int32 block
ids, per-request arrays, packed ancestor rows).  The derived properties,
``slot_mapping``, ``validate_block_tables`` and the backend's step plan all
read those arrays, so a step's tuples are walked once.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch
from torch import Tensor

from light_vllm_amd.facts import StepFacts, parse_fields
from light_vllm_amd.interfaces import QueryLayout


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
        # One native call: the fields as tuples with their defaults (empty
        # reserved -> each layout's query count, empty readonly -> zeros),
        # every field rule in order, and the step facts.
        fields, facts = parse_fields(self.block_tables, self.num_computed_tokens, self.query_layouts,
                                     self.num_reserved_query_tokens, self.num_readonly_prefix_blocks)
        put = object.__setattr__
        put(self, "block_tables", fields[0])
        put(self, "num_computed_tokens", fields[1])
        put(self, "query_layouts", fields[2])
        put(self, "num_reserved_query_tokens", fields[3])
        put(self, "num_readonly_prefix_blocks", fields[4])
        put(self, "facts", facts)

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
