"""Per-step batch facts of a packed paged-attention batch.

Restates the behaviour of light-vllm's ``PagedAttentionMetadata``
(src/light_vllm/runtime/execution/paged_attention.py:18-206): the same fields,
defaults, derived properties, validation rules and error messages.  The HIP
backend reads a metadata object only through these attributes, so light-vllm's
own class can be passed in its place.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import Tensor

from light_vllm_amd.errors import KVCacheError
from light_vllm_amd.interfaces import QueryLayout
from light_vllm_amd.layout import is_linear, query_visibility


@dataclass(frozen=True, slots=True)
class PagedAttentionMetadata:
    """Block tables, computed-token counts and query layouts of one step."""

    block_tables: tuple[tuple[int, ...], ...]
    num_computed_tokens: tuple[int, ...]
    query_layouts: tuple[QueryLayout, ...]
    # Actual queries plus the scheduler's reserved, possibly unused, slots.
    num_reserved_query_tokens: tuple[int, ...] = ()
    num_readonly_prefix_blocks: tuple[int, ...] = ()

    def __post_init__(self) -> None:
        block_tables = tuple(tuple(table) for table in self.block_tables)
        computed = tuple(self.num_computed_tokens)
        layouts = tuple(self.query_layouts)
        reserved = tuple(self.num_reserved_query_tokens)
        readonly = tuple(self.num_readonly_prefix_blocks)
        num_requests = len(block_tables)
        if num_requests == 0:
            raise ValueError("paged attention metadata must contain at least one request")
        if len(computed) != num_requests or len(layouts) != num_requests:
            raise ValueError("paged attention metadata fields must have the same batch size")
        if not reserved:
            reserved = tuple(len(layout) for layout in layouts)
        if len(reserved) != num_requests:
            raise ValueError("reserved query counts must have the same batch size")
        if not readonly:
            readonly = (0,) * num_requests
        if len(readonly) != num_requests:
            raise ValueError("readonly prefix counts must have the same batch size")
        if any(type(value) is not int or value < 0 for value in computed):
            raise ValueError("computed-token counts must be non-negative integers")
        if any(type(value) is not int or value < len(layout) for value, layout in zip(reserved, layouts)):
            raise ValueError("reserved query counts must cover every actual query")
        if any(type(value) is not int or value < 0 for value in readonly):
            raise ValueError("readonly prefix counts must be non-negative integers")
        if any(type(b) is not int or b < 0 for table in block_tables for b in table):
            raise ValueError("block tables must contain non-negative integers")
        object.__setattr__(self, "block_tables", block_tables)
        object.__setattr__(self, "num_computed_tokens", computed)
        object.__setattr__(self, "query_layouts", layouts)
        object.__setattr__(self, "num_reserved_query_tokens", reserved)
        object.__setattr__(self, "num_readonly_prefix_blocks", readonly)

    @property
    def batch_size(self) -> int:
        return len(self.block_tables)

    @property
    def query_lengths(self) -> tuple[int, ...]:
        return tuple(len(layout) for layout in self.query_layouts)

    @property
    def query_start_loc(self) -> tuple[int, ...]:
        starts = [0]
        for length in self.query_lengths:
            starts.append(starts[-1] + length)
        return tuple(starts)

    @property
    def num_query_tokens(self) -> int:
        return sum(self.query_lengths)

    @property
    def has_only_linear_queries(self) -> bool:
        return all(is_linear(layout) for layout in self.query_layouts)

    @property
    def request_indices(self) -> tuple[int, ...]:
        out: list[int] = []
        for index, length in enumerate(self.query_lengths):
            out.extend([index] * length)
        return tuple(out)

    def _check_coverage(self, table: tuple[int, ...], computed: int, reserved: int, block_size: int) -> None:
        required = -(-(computed + reserved) // block_size)
        if len(table) < required:
            raise KVCacheError("block table does not cover all scheduled tokens")
        if len(table) > required:
            raise KVCacheError("block table contains unused physical blocks")

    def slot_mapping(self, *, block_size: int, device: torch.device) -> Tensor:
        """Physical slot of every packed query token: table[p // bs] * bs + p % bs."""

        mapping: list[int] = []
        for table, computed, layout, reserved in zip(
            self.block_tables, self.num_computed_tokens, self.query_layouts, self.num_reserved_query_tokens
        ):
            self._check_coverage(table, computed, reserved, block_size)
            for position in range(computed, computed + len(layout)):
                mapping.append(table[position // block_size] * block_size + position % block_size)
        return torch.tensor(mapping, dtype=torch.long, device=device)

    def validate_block_tables(self, *, num_blocks: int, block_size: int) -> None:
        """Prove the tables safe to read and write this step (rules of the reference)."""

        owners: dict[int, tuple[int, bool]] = {}
        for table, computed, reserved, num_readonly in zip(
            self.block_tables,
            self.num_computed_tokens,
            self.num_reserved_query_tokens,
            self.num_readonly_prefix_blocks,
        ):
            self._check_coverage(table, computed, reserved, block_size)
            if any(block_id >= num_blocks for block_id in table):
                raise KVCacheError("block table contains an out-of-range physical block")
            if num_readonly > len(table) or num_readonly * block_size > computed:
                raise KVCacheError("readonly prefix blocks exceed the computed prefix")
            if len(set(table)) != len(table):
                raise KVCacheError("block table aliases a physical block within one request")
            for logical_index, block_id in enumerate(table):
                readonly = logical_index < num_readonly
                previous = owners.get(block_id)
                if previous is not None and (
                    previous[0] != logical_index or not previous[1] or not readonly
                ):
                    raise KVCacheError("block tables alias a physical block across requests")
                owners[block_id] = (logical_index, readonly)

    def visibility_tensor(self, *, device: torch.device) -> tuple[Tensor, Tensor]:
        """Row-major q x q ancestor masks of all requests, concatenated, and their starts."""

        flat: list[bool] = []
        starts = [0]
        for layout in self.query_layouts:
            for row in query_visibility(layout):
                flat.extend(row)
            starts.append(len(flat))
        return (
            torch.tensor(flat, dtype=torch.bool, device=device),
            torch.tensor(starts, dtype=torch.int32, device=device),
        )

    def request_indices_tensor(self, *, device: torch.device) -> Tensor:
        return torch.tensor(self.request_indices, dtype=torch.int32, device=device)

    def visible_logical_positions(self, row: int) -> tuple[tuple[int, ...], ...]:
        """Logical key positions every query of request ``row`` may read."""

        computed = self.num_computed_tokens[row]
        prefix = tuple(range(computed))
        return tuple(
            prefix + tuple(computed + j for j, seen in enumerate(visible) if seen)
            for visible in query_visibility(self.query_layouts[row])
        )
