"""Types the paged-KV path shares with its callers.

Restated with the behaviour of light-vllm's definitions so the backend can run
stand-alone; when plugged into light-vllm the real classes are passed instead
and only the attributes used here are read.

* ``AttentionLayerSpec`` / ``ModelKVCacheSpec`` / ``AttentionContext``:
  src/light_vllm/modeling/attention/interfaces.py:9-62
* ``QueryLayout`` / ``DraftTree``: src/light_vllm/runtime/execution/interfaces.py:53-97
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Protocol

from torch import Tensor


@dataclass(frozen=True, slots=True)
class AttentionLayerSpec:
    """Logical K/V shape of one attention layer."""

    layer_id: str
    num_query_heads: int
    num_kv_heads: int
    head_size: int

    def __post_init__(self) -> None:
        if not self.layer_id:
            raise ValueError("layer_id must not be empty")
        for name, value in (
            ("num_query_heads", self.num_query_heads),
            ("num_kv_heads", self.num_kv_heads),
            ("head_size", self.head_size),
        ):
            if type(value) is not int or value <= 0:
                raise ValueError(f"{name} must be a positive integer")
        if self.num_query_heads % self.num_kv_heads != 0:
            raise ValueError("num_query_heads must be divisible by num_kv_heads")


@dataclass(frozen=True, slots=True)
class ModelKVCacheSpec:
    """K/V shapes of every cacheable attention layer of a model."""

    layers: tuple[AttentionLayerSpec, ...]

    def __post_init__(self) -> None:
        layers = tuple(self.layers)
        layer_ids = tuple(layer.layer_id for layer in layers)
        if not layers:
            raise ValueError("model KV cache spec must contain at least one layer")
        if len(set(layer_ids)) != len(layer_ids):
            raise ValueError("attention layer IDs must be unique")
        object.__setattr__(self, "layers", layers)


class AttentionContext(Protocol):
    """What a model attention layer calls once per layer per step."""

    def forward(
        self,
        layer_id: str,
        query: Tensor,
        key: Tensor,
        value: Tensor,
        *,
        scale: float,
    ) -> Tensor:
        """Write this step's K/V, then return attention with ``query``'s shape."""
        ...


@dataclass(frozen=True, slots=True)
class QueryLayout:
    """Parent of every query of one request inside a model step (-1 = root)."""

    parent_indices: tuple[int, ...]

    def __post_init__(self) -> None:
        parent_indices = tuple(self.parent_indices)
        if not parent_indices:
            raise ValueError("query layout must not be empty")
        for index, parent in enumerate(parent_indices):
            if type(parent) is not int or not -1 <= parent < index:
                raise ValueError("each query parent must be -1 or precede its child")
        object.__setattr__(self, "parent_indices", parent_indices)

    def __len__(self) -> int:
        return len(self.parent_indices)


@dataclass(frozen=True, slots=True)
class DraftTree:
    """Draft tree flattened parent-first."""

    token_ids: tuple[int, ...]
    parent_indices: tuple[int, ...]

    def __post_init__(self) -> None:
        token_ids = tuple(self.token_ids)
        parent_indices = tuple(self.parent_indices)
        if len(token_ids) != len(parent_indices):
            raise ValueError("draft tokens and parents must have the same length")
        if any(type(token_id) is not int or token_id < 0 for token_id in token_ids):
            raise ValueError("draft tokens must be non-negative integers")
        siblings: set[tuple[int, int]] = set()
        for index, (token_id, parent) in enumerate(zip(token_ids, parent_indices, strict=True)):
            if type(parent) is not int or not -1 <= parent < index:
                raise ValueError("each draft parent must be -1 or precede its child")
            sibling = (parent, token_id)
            if sibling in siblings:
                raise ValueError("draft siblings must use distinct token IDs")
            siblings.add(sibling)
        object.__setattr__(self, "token_ids", token_ids)
        object.__setattr__(self, "parent_indices", parent_indices)

    def __len__(self) -> int:
        return len(self.token_ids)
