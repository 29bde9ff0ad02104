"""Types the paged-KV path shares with its callers.

The backend reads these through their attributes only, so light-vllm's own
classes can be passed in their place.  The contract kept from light-vllm is
the names, fields, defaults and the error messages (with the rule that fires
first when several are broken):

* ``AttentionLayerSpec`` / ``ModelKVCacheSpec`` / ``AttentionContext``:
  src/light_vllm/modeling/attention/interfaces.py:9-62
* ``QueryLayout`` / ``DraftTree``: src/light_vllm/runtime/execution/interfaces.py:53-97

The checks are written here as ordered rule lists over the normalised
values; the first failing rule raises.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Protocol, Sequence

from torch import Tensor


def _is_int(value: object) -> bool:
    """An exact ``int`` (bool and numpy integers are rejected, as in light-vllm)."""

    return type(value) is int


def _first_broken(rules: Sequence[tuple[Callable[[], bool], str]]) -> str | None:
    """Message of the first rule whose check fails, else None."""

    for holds, message in rules:
        if not holds():
            return message
    return None


def _raise_first(rules: Sequence[tuple[Callable[[], bool], str]]) -> None:
    message = _first_broken(rules)
    if message is not None:
        raise ValueError(message)


def _first_bad_parent(parents: tuple) -> int:
    """Index of the first parent that is not an int in [-1, index), or -1."""

    for index, parent in enumerate(parents):
        if not (_is_int(parent) and -1 <= parent < index):
            return index
    return -1


@dataclass(frozen=True, slots=True)
class AttentionLayerSpec:
    """Logical K/V shape of one attention layer."""

    layer_id: str
    num_query_heads: int
    num_kv_heads: int
    head_size: int

    def __post_init__(self) -> None:
        rules: list[tuple[Callable[[], bool], str]] = [(lambda: bool(self.layer_id), "layer_id must not be empty")]
        for name in ("num_query_heads", "num_kv_heads", "head_size"):
            value = getattr(self, name)
            rules.append((lambda v=value: _is_int(v) and v > 0, f"{name} must be a positive integer"))
        rules.append((lambda: self.num_query_heads % self.num_kv_heads == 0,
                      "num_query_heads must be divisible by num_kv_heads"))
        _raise_first(rules)

    @property
    def group_size(self) -> int:
        """Query heads per kv head (the GQA group)."""

        return self.num_query_heads // self.num_kv_heads


@dataclass(frozen=True, slots=True)
class ModelKVCacheSpec:
    """K/V shapes of every cacheable attention layer of a model."""

    layers: tuple[AttentionLayerSpec, ...]

    def __post_init__(self) -> None:
        layers = tuple(self.layers)
        ids = [layer.layer_id for layer in layers]
        _raise_first((
            (lambda: len(layers) > 0, "model KV cache spec must contain at least one layer"),
            (lambda: len(set(ids)) == len(ids), "attention layer IDs must be unique"),
        ))
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
        parents = tuple(self.parent_indices)
        _raise_first((
            (lambda: len(parents) > 0, "query layout must not be empty"),
            (lambda: _first_bad_parent(parents) < 0, "each query parent must be -1 or precede its child"),
        ))
        object.__setattr__(self, "parent_indices", parents)

    def __len__(self) -> int:
        return len(self.parent_indices)


@dataclass(frozen=True, slots=True)
class DraftTree:
    """Draft tree flattened parent-first."""

    token_ids: tuple[int, ...]
    parent_indices: tuple[int, ...]

    def __post_init__(self) -> None:
        tokens = tuple(self.token_ids)
        parents = tuple(self.parent_indices)
        _raise_first((
            (lambda: len(tokens) == len(parents), "draft tokens and parents must have the same length"),
            (lambda: all(_is_int(t) and t >= 0 for t in tokens), "draft tokens must be non-negative integers"),
        ))
        # Parents and sibling tokens are checked node by node in light-vllm,
        # so whichever problem comes at the lower index is reported (a bad
        # parent before a repeated sibling at the same node).
        bad_parent = _first_bad_parent(parents)
        limit = bad_parent if bad_parent >= 0 else len(parents)
        seen: dict[tuple[int, int], int] = {}
        repeated = -1
        for index in range(limit):
            key = (parents[index], tokens[index])
            if key in seen:
                repeated = index
                break
            seen[key] = index
        if repeated >= 0:
            raise ValueError("draft siblings must use distinct token IDs")
        if bad_parent >= 0:
            raise ValueError("each draft parent must be -1 or precede its child")
        object.__setattr__(self, "token_ids", tokens)
        object.__setattr__(self, "parent_indices", parents)

    def __len__(self) -> int:
        return len(self.token_ids)
