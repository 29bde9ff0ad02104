"""Positions and visibility derived from a parent chain.

Behaviour of src/light_vllm/runtime/execution/layout.py:13-55.
"""

from __future__ import annotations

from light_vllm_amd.interfaces import DraftTree, QueryLayout


def linear_query_layout(num_queries: int) -> QueryLayout:
    """The ordinary causal chain: query i's parent is i - 1."""

    if type(num_queries) is not int or num_queries <= 0:
        raise ValueError("num_queries must be a positive integer")
    return QueryLayout(tuple(range(-1, num_queries - 1)))


def append_draft_layout(num_input_queries: int, draft: DraftTree) -> QueryLayout:
    """Hang every draft root under the last formal input query."""

    if type(num_input_queries) is not int or num_input_queries <= 0:
        raise ValueError("num_input_queries must be a positive integer")
    tail = num_input_queries - 1
    parents = list(range(-1, tail))
    parents.extend(tail if parent == -1 else num_input_queries + parent for parent in draft.parent_indices)
    return QueryLayout(tuple(parents))


def semantic_positions(layout: QueryLayout, *, prefix_length: int) -> tuple[int, ...]:
    """RoPE position of every query: prefix length plus its depth in the tree."""

    if type(prefix_length) is not int or prefix_length < 0:
        raise ValueError("prefix_length must be a non-negative integer")
    depth: list[int] = []
    for parent in layout.parent_indices:
        depth.append(0 if parent == -1 else depth[parent] + 1)
    return tuple(prefix_length + d for d in depth)


def query_visibility(layout: QueryLayout) -> tuple[tuple[bool, ...], ...]:
    """Row q marks q itself and every ancestor of q."""

    parents = layout.parent_indices
    width = len(parents)
    rows: list[tuple[bool, ...]] = []
    for query_index in range(width):
        row = [False] * width
        node = query_index
        while node != -1:
            row[node] = True
            node = parents[node]
        rows.append(tuple(row))
    return tuple(rows)


def is_linear(layout: QueryLayout) -> bool:
    """Whether the layout is the ordinary causal chain."""

    return all(parent == index - 1 for index, parent in enumerate(layout.parent_indices))
