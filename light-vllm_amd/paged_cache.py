"""Physical paged K/V pool on an MI355X, with HIP append, compact and block copy.

Restates light-vllm's ``PagedKVCache`` (src/light_vllm/runtime/execution/
paged_cache.py:30-338): same config, same per-layer layout
``[num_blocks, block_size, num_kv_heads, head_size]`` (separate K and V
tensors), same validation rules and messages.  The data movement runs in the
gfx950 kernels of ``liblvamd_hip.so``; there is no PyTorch fallback, and a
cache on a non-GPU device is rejected.

``hip_compact`` and ``hip_block_copy`` work on any cache object exposing the
reference's public surface (``config``, ``model_spec.layers``, ``layer(id)``),
so light-vllm's own ``PagedKVCache`` can use them unchanged.
"""

from __future__ import annotations

import weakref
from dataclasses import dataclass

import torch
from torch import Tensor

from light_vllm_amd import native
from light_vllm_amd.errors import KVCacheError
from light_vllm_amd.interfaces import AttentionLayerSpec, ModelKVCacheSpec
from light_vllm_amd.plan import table_proven

_DTYPE_CODES = {torch.float32: native.DTYPE_F32, torch.float16: native.DTYPE_F16, torch.bfloat16: native.DTYPE_BF16}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError as exc:
        raise KVCacheError(f"HIP paged KV supports float32, float16 and bfloat16, not {dtype}") from exc


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream(device: torch.device) -> int:
    """The current HIP stream of ``device`` as a raw handle (torch's own
    accessor when present: it skips building a Stream object per call)."""

    if _raw_stream is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(index)
    return torch.cuda.current_stream(device).cuda_stream


@dataclass(frozen=True, slots=True)
class PagedKVCacheConfig:
    """Number and size of physical blocks, dtype and device of the pool."""

    num_blocks: int
    block_size: int
    dtype: torch.dtype = torch.float32
    device: str | torch.device = "cpu"

    def __post_init__(self) -> None:
        if type(self.num_blocks) is not int or self.num_blocks <= 0:
            raise ValueError("num_blocks must be a positive integer")
        if type(self.block_size) is not int or self.block_size <= 0:
            raise ValueError("block_size must be a positive integer")
        if not self.dtype.is_floating_point:
            raise ValueError("KV cache dtype must be floating point")
        object.__setattr__(self, "device", torch.device(self.device))

    def plan(self, model_spec: ModelKVCacheSpec) -> "PagedKVCacheConfig":
        return self


def kv_cache_bytes_per_block(model_spec: ModelKVCacheSpec, *, block_size: int, dtype: torch.dtype) -> int:
    """Bytes of one physical block across all layers, K and V."""

    per_token = sum(2 * layer.num_kv_heads * layer.head_size for layer in model_spec.layers)
    return block_size * per_token * torch.empty((), dtype=dtype).element_size()


@dataclass(frozen=True, slots=True)
class PagedLayerCache:
    """One layer's K and V, each ``[block, offset, kv_head, head_size]``."""

    keys: Tensor
    values: Tensor


@dataclass(frozen=True, slots=True)
class PagedKVWriteMapping:
    """Physical write slots of one step, reused by every layer."""

    slots: Tensor
    num_query_tokens: int
    source_indices: Tensor | None = None


class _LayerPointers:
    """Device arrays of per-layer K and V base addresses, grouped by row size."""

    def __init__(self, cache) -> None:
        device = cache.config.device
        groups: dict[int, list[tuple[int, int]]] = {}
        for spec in cache.model_spec.layers:
            layer = cache.layer(spec.layer_id)
            row_bytes = spec.num_kv_heads * spec.head_size * layer.keys.element_size()
            groups.setdefault(row_bytes, []).append((layer.keys.data_ptr(), layer.values.data_ptr()))
        self.groups: list[tuple[int, int, Tensor]] = []
        for row_bytes, ptrs in groups.items():
            table = torch.tensor(ptrs, dtype=torch.int64).t().contiguous().to(device)
            self.groups.append((row_bytes, len(ptrs), table))


_POINTER_CACHE: "weakref.WeakKeyDictionary[object, _LayerPointers]" = weakref.WeakKeyDictionary()


def _layer_pointers(cache) -> _LayerPointers:
    """Per-cache pointer tables, built on first use and dropped with the cache."""

    found = _POINTER_CACHE.get(cache)
    if found is None:
        found = _LayerPointers(cache)
        _POINTER_CACHE[cache] = found
    return found


def _require_gpu(cache) -> None:
    if cache.config.device.type != "cuda":
        raise KVCacheError("the HIP paged KV path requires a GPU KV cache")


def hip_append(cache, layer_id: str, key: Tensor, value: Tensor, slots: Tensor) -> None:
    """``flatK[slots[t]] = key[t]``, ``flatV[slots[t]] = value[t]`` on the current stream.

    ``slots`` is int64 with one entry per token (negative = skip).
    """

    layer = cache.layer(layer_id)
    spec = cache.layer_spec(layer_id)
    if key.stride(2) != 1 or value.stride(2) != 1:
        key = key.contiguous()
        value = value.contiguous()
    lib = native.load()
    status = lib.lvamd_kv_append(
        key.data_ptr(), key.stride(0), key.stride(1),
        value.data_ptr(), value.stride(0), value.stride(1),
        layer.keys.data_ptr(), layer.values.data_ptr(),
        slots.data_ptr(), slots.numel(),
        spec.num_kv_heads, spec.head_size, dtype_code(key.dtype),
        current_stream(key.device),
    )
    native.check(status, "lvamd_kv_append")


def hip_append_rotary(cache, layer_id: str, query: Tensor, key: Tensor, value: Tensor,
                      rotary: tuple[Tensor, Tensor], slots: Tensor) -> Tensor:
    """Rotate ``query`` and ``key`` (Qwen2's half rotation, rounded as
    apply_rotary's PyTorch path rounds it) and append: ``flatK[slots[t]] =
    rotate(key[t])``, ``flatV[slots[t]] = value[t]``; returns the rotated
    queries as a new tensor.  One kernel on the current stream.

    apply_rotary: src/light_vllm/modeling/models/_qwen2_kernels.py:205-245;
    append: src/light_vllm/runtime/execution/paged_cache.py:209-248.
    """

    spec = cache.layer_spec(layer_id)
    cosines, sines = rotary
    tokens = query.shape[0]
    for name, t in (("cosines", cosines), ("sines", sines)):
        if not isinstance(t, Tensor) or t.dim() != 2 or tuple(t.shape) != (tokens, spec.head_size):
            raise KVCacheError(f"rotary {name} must have shape [{tokens}, {spec.head_size}]")
        if t.dtype != query.dtype or t.device != query.device:
            raise KVCacheError(f"rotary {name} dtype and device must match the query")
    if cosines.stride(1) != 1:
        cosines = cosines.contiguous()
    if sines.stride(1) != 1:
        sines = sines.contiguous()
    if query.stride(2) != 1:
        query = query.contiguous()
    if key.stride(2) != 1 or value.stride(2) != 1:
        key = key.contiguous()
        value = value.contiguous()
    layer = cache.layer(layer_id)
    rotated = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    lib = native.load()
    status = lib.lvamd_kv_append_rotary(
        query.data_ptr(), query.stride(0), query.stride(1),
        rotated.data_ptr(), rotated.stride(0), rotated.stride(1),
        key.data_ptr(), key.stride(0), key.stride(1),
        value.data_ptr(), value.stride(0), value.stride(1),
        cosines.data_ptr(), cosines.stride(0), sines.data_ptr(), sines.stride(0),
        layer.keys.data_ptr(), layer.values.data_ptr(), slots.data_ptr(), slots.numel(),
        spec.num_query_heads, spec.num_kv_heads, spec.head_size, dtype_code(query.dtype),
        current_stream(query.device),
    )
    native.check(status, "lvamd_kv_append_rotary")
    return rotated


def compact_slots(
    config,
    block_ids: tuple[int, ...],
    *,
    num_computed_tokens: int,
    num_query_tokens: int,
    num_reserved_query_tokens: int,
    retained_query_indices: tuple[int, ...],
    num_readonly_prefix_blocks: int = 0,
) -> tuple[tuple[int, ...], tuple[int, ...]]:
    """Validate a compact request and return (source slots, target slots).

    Rules and messages of PagedKVCache.compact (paged_cache.py:269-312).
    """

    block_ids = tuple(block_ids)
    retained = tuple(retained_query_indices)
    counts = (num_computed_tokens, num_query_tokens, num_reserved_query_tokens, num_readonly_prefix_blocks)
    if any(type(v) is not int or v < 0 for v in counts):
        raise ValueError("paged compact counts must be non-negative integers")
    if num_reserved_query_tokens < num_query_tokens:
        raise ValueError("reserved query tokens must cover every actual query")
    if any(type(i) is not int or i < 0 for i in retained):
        raise ValueError("retained query indices must be non-negative integers")
    if len(set(retained)) != len(retained):
        raise ValueError("retained query indices must be unique")
    if any(i >= num_query_tokens for i in retained):
        raise KVCacheError("retained query index exceeds the paged KV tail")
    bs = config.block_size
    required = (num_computed_tokens + num_reserved_query_tokens + bs - 1) // bs
    if len(block_ids) != required:
        raise KVCacheError("block table does not exactly cover the reserved query slots")
    # Every id an int (not a bool or numpy scalar) in [0, num_blocks), none
    # repeated; checked with C-level passes (map/min/max/set) since tables run
    # to thousands of ids, and skipped for a table object that the step's
    # attention context has already proven (plan.table_proven).
    if not table_proven(block_ids, config.num_blocks):
        if block_ids and (
            set(map(type, block_ids)) != {int} or min(block_ids) < 0 or max(block_ids) >= config.num_blocks
        ):
            raise KVCacheError("block table contains an invalid physical block")
        if len(set(block_ids)) != len(block_ids):
            raise KVCacheError("block table aliases a physical block within one request")
    if num_readonly_prefix_blocks * bs > num_computed_tokens:
        raise KVCacheError("readonly prefix blocks exceed the computed prefix")

    def slot(position: int) -> int:
        return block_ids[position // bs] * bs + position % bs

    sources = tuple(slot(num_computed_tokens + i) for i in retained)
    targets = tuple(slot(num_computed_tokens + i) for i in range(len(retained)))
    return sources, targets


def hip_compact(cache, block_ids: tuple[int, ...], **kwargs) -> int:
    """Move the retained query K/V to the contiguous formal tail of every layer.

    Returns the number of tokens whose slot changed (0 = nothing written).
    Pairs whose source equals their target are dropped before the copy: such
    a slot is neither read nor written by any other pair (targets are unique
    and sources are unique), so dropping it leaves the result unchanged.
    """

    _require_gpu(cache)
    sources, targets = compact_slots(cache.config, block_ids, **kwargs)
    moved = [(s, t) for s, t in zip(sources, targets) if s != t]
    _launch_compact(cache, moved)
    return len(moved)


def hip_compact_many(cache, requests) -> tuple[int, ...]:
    """``hip_compact`` for several requests of one step in a single launch.

    Each request is a mapping of ``hip_compact``'s keyword arguments
    (``block_ids``, ``num_computed_tokens``, ...), validated exactly as a
    single compact; destinations must be unique across the batch (every
    source is read before any destination is written, as for one request).
    Returns each request's moved-token count.
    """

    _require_gpu(cache)
    moved: list[tuple[int, int]] = []
    counts = []
    for request in requests:
        kwargs = dict(request)
        block_ids = kwargs.pop("block_ids")
        sources, targets = compact_slots(cache.config, tuple(block_ids), **kwargs)
        pairs = [(s, t) for s, t in zip(sources, targets) if s != t]
        counts.append(len(pairs))
        moved += pairs
    if len({t for _, t in moved}) != len(moved):
        raise KVCacheError("compact requests of one step must not write the same slot")
    _launch_compact(cache, moved)
    return tuple(counts)


def _launch_compact(cache, moved: list[tuple[int, int]]) -> None:
    if not moved:
        return
    device = cache.config.device
    pairs = torch.tensor(moved, dtype=torch.int64).t().contiguous()
    if device.type == "cuda":
        pairs = pairs.pin_memory()
    pairs = pairs.to(device, non_blocking=True)
    lib = native.load()
    stream = current_stream(device)
    n = len(moved)
    for row_bytes, num_layers, ptrs in _layer_pointers(cache).groups:
        ws_bytes = lib.lvamd_kv_compact_workspace_size(n, num_layers, row_bytes)
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device) if ws_bytes else None
        status = lib.lvamd_kv_compact(
            ptrs[0].data_ptr(), ptrs[1].data_ptr(), num_layers, row_bytes,
            pairs[0].data_ptr(), pairs[1].data_ptr(), n,
            workspace.data_ptr() if workspace is not None else None, ws_bytes, stream,
        )
        native.check(status, "lvamd_kv_compact")


def hip_block_copy(cache, src_blocks, dst_blocks) -> None:
    """Copy-on-write: block ``dst_blocks[i]`` of every layer becomes a copy of ``src_blocks[i]``.

    No light-vllm counterpart (its prefix cache shares only complete read-only
    pages).  Sources and destinations must be disjoint and destinations unique.
    """

    _require_gpu(cache)
    src = tuple(src_blocks)
    dst = tuple(dst_blocks)
    if len(src) != len(dst):
        raise ValueError("block copy needs one destination per source")
    num_blocks = cache.config.num_blocks
    both = src + dst
    if both and (set(map(type, both)) != {int} or min(both) < 0 or max(both) >= num_blocks):
        raise KVCacheError("block copy names an invalid physical block")
    if len(set(dst)) != len(dst):
        raise KVCacheError("block copy writes the same physical block twice")
    if set(src) & set(dst):
        raise KVCacheError("block copy sources and destinations must be disjoint")
    if not src:
        return
    device = cache.config.device
    pairs = torch.tensor((src, dst), dtype=torch.int64)
    if device.type == "cuda":
        pairs = pairs.pin_memory()
    pairs = pairs.to(device, non_blocking=True)
    lib = native.load()
    stream = current_stream(device)
    bs = cache.config.block_size
    for row_bytes, num_layers, ptrs in _layer_pointers(cache).groups:
        status = lib.lvamd_kv_block_copy(
            ptrs[0].data_ptr(), ptrs[1].data_ptr(), num_layers, row_bytes * bs,
            pairs[0].data_ptr(), pairs[1].data_ptr(), len(src), stream,
        )
        native.check(status, "lvamd_kv_block_copy")


class PagedKVCache:
    """Per-layer K/V pools shared by all requests, addressed by block id."""

    def __init__(self, model_spec: ModelKVCacheSpec, config: PagedKVCacheConfig) -> None:
        if config.device.type != "cuda":
            raise KVCacheError("the HIP paged KV cache requires a GPU (cuda) device")
        dtype_code(config.dtype)
        self._model_spec = model_spec
        self._config = config
        self._layer_specs = {layer.layer_id: layer for layer in model_spec.layers}
        self._layers = {layer.layer_id: self._allocate_layer(layer) for layer in model_spec.layers}

    @property
    def config(self) -> PagedKVCacheConfig:
        return self._config

    @property
    def model_spec(self) -> ModelKVCacheSpec:
        return self._model_spec

    def layer_spec(self, layer_id: str) -> AttentionLayerSpec:
        try:
            return self._layer_specs[layer_id]
        except KeyError as exc:
            raise KVCacheError(f"KV cache layer {layer_id!r} was not found") from exc

    def layer(self, layer_id: str) -> PagedLayerCache:
        try:
            return self._layers[layer_id]
        except KeyError as exc:
            raise KVCacheError(f"KV cache layer {layer_id!r} was not found") from exc

    @torch.inference_mode()
    def prepare_write(self, slot_mapping: Tensor, *, validate: bool = True) -> PagedKVWriteMapping:
        """Normalise one step's slot mapping for reuse by all layers (paged_cache.py:165-206)."""

        if slot_mapping.ndim != 1:
            raise KVCacheError("slot mapping must have one entry per packed query token")
        if slot_mapping.device != self._config.device:
            raise KVCacheError("slot mapping device must match the cache")
        flat = slot_mapping.flatten()
        if not validate:
            return PagedKVWriteMapping(slots=flat.to(torch.long), num_query_tokens=flat.numel())
        active = flat >= 0
        source_indices = torch.nonzero(active, as_tuple=False).flatten()
        slots = flat.index_select(0, source_indices).to(torch.long)
        if slots.numel():
            num_slots = self._config.num_blocks * self._config.block_size
            if int(slots.min()) < 0 or int(slots.max()) >= num_slots:
                raise KVCacheError("slot mapping contains an out-of-range physical slot")
            if slots.unique().numel() != slots.numel():
                raise KVCacheError("slot mapping must not write the same physical slot twice")
        return PagedKVWriteMapping(
            slots=slots,
            num_query_tokens=flat.numel(),
            source_indices=None if source_indices.numel() == flat.numel() else source_indices,
        )

    @torch.inference_mode()
    def write_prepared(self, layer_id: str, key: Tensor, value: Tensor, mapping: PagedKVWriteMapping) -> None:
        """Write K/V through a prepared mapping (paged_cache.py:209-248), on the HIP append kernel."""

        self.layer(layer_id)
        spec = self.layer_spec(layer_id)
        tail = (spec.num_kv_heads, spec.head_size)
        if key.ndim != 3 or tuple(key.shape[1:]) != tail:
            raise KVCacheError("paged KV update must have shape [tokens, kv_heads, head_size]")
        if value.shape != key.shape:
            raise KVCacheError("paged K/V updates must have the same shape")
        if mapping.num_query_tokens != key.shape[0]:
            raise KVCacheError("slot mapping must have one entry per query token")
        if key.dtype != self._config.dtype or key.device != self._config.device:
            raise KVCacheError("paged KV update dtype and device must match the cache")
        if value.dtype != key.dtype or value.device != key.device:
            raise KVCacheError("paged K/V updates must use the same dtype and device")
        if mapping.slots.device != self._config.device or (
            mapping.source_indices is not None and mapping.source_indices.device != self._config.device
        ):
            raise KVCacheError("prepared slot mapping device must match the cache")
        if mapping.slots.numel() == 0:
            return
        slots = mapping.slots
        if mapping.source_indices is not None:
            dense = torch.full((mapping.num_query_tokens,), -1, dtype=torch.long, device=slots.device)
            dense.index_copy_(0, mapping.source_indices, slots)
            slots = dense
        hip_append(self, layer_id, key, value, slots.contiguous())

    @torch.inference_mode()
    def write(self, layer_id: str, key: Tensor, value: Tensor, slot_mapping: Tensor) -> None:
        """Write the active tokens' K/V to their physical slots."""

        self.write_prepared(layer_id, key, value, self.prepare_write(slot_mapping))

    @torch.inference_mode()
    def compact(
        self,
        block_ids: tuple[int, ...],
        *,
        num_computed_tokens: int,
        num_query_tokens: int,
        num_reserved_query_tokens: int,
        retained_query_indices: tuple[int, ...],
        num_readonly_prefix_blocks: int = 0,
    ) -> int:
        """Move the accepted path to the contiguous formal tail (paged_cache.py:257-326)."""

        return hip_compact(
            self,
            block_ids,
            num_computed_tokens=num_computed_tokens,
            num_query_tokens=num_query_tokens,
            num_reserved_query_tokens=num_reserved_query_tokens,
            retained_query_indices=retained_query_indices,
            num_readonly_prefix_blocks=num_readonly_prefix_blocks,
        )

    @torch.inference_mode()
    def compact_many(self, requests) -> tuple[int, ...]:
        """``compact`` for every request of a step in one launch (one mapping of
        ``compact``'s arguments, with ``block_ids``, per request)."""

        return hip_compact_many(self, requests)

    @torch.inference_mode()
    def copy_blocks(self, src_blocks, dst_blocks) -> None:
        """Copy-on-write of whole blocks across every layer (no reference counterpart)."""

        hip_block_copy(self, src_blocks, dst_blocks)

    def _allocate_layer(self, spec: AttentionLayerSpec) -> PagedLayerCache:
        shape = (self._config.num_blocks, self._config.block_size, spec.num_kv_heads, spec.head_size)
        return PagedLayerCache(
            keys=torch.empty(shape, dtype=self._config.dtype, device=self._config.device),
            values=torch.empty(shape, dtype=self._config.dtype, device=self._config.device),
        )
